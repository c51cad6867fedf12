/* p0k.h — C ABI of the MI355X-native `gemm` path of p0pc0rn-kernels.
 *
 * One library (libp0k.so, HIP on gfx950) replaces the WebGPU runtime and the WGSL GEMM generator of the reference:
 *
 *   reference (JavaScript / WebGPU)                         this ABI
 *   -------------------------------------------------------  ---------------------------------------------
 *   createGpu(opts)            src/core/gpu.js:15-20         p0k_ctx_create / p0k_ctx_destroy
 *   Gpu.buffer(size)           src/core/gpu.js:87-110        p0k_alloc   (zeroed, 16-byte rounded, pooled)
 *   Gpu.free(buf)              src/core/gpu.js:112-121       p0k_free
 *   Gpu.upload(data,..,dst)    src/core/gpu.js:141-148       p0k_upload
 *   Gpu.read(buf, off, size)   src/core/gpu.js:150-170       p0k_download (blocks until the stream is done)
 *   Gpu.done()                 src/core/gpu.js:171-176       p0k_sync
 *   Gpu.poolStats/drainPool    src/core/gpu.js:134-137       p0k_pool_stats / p0k_drain_pool
 *   gemm(gpu, args)            src/ops/gemm.js:268-327       p0k_gemm (args: p0k_gemm_args, the fields of GemmArgs,
 *                                                            types/index.d.ts:128-150, and of the uniform P, gemm.js:39-41)
 *   argument errors of gemm    src/ops/gemm.js:31,271,283,313 p0k_gemm_check (host only, never touches the GPU)
 *   rowstats(gpu, a)           src/ops/misc.js:16-44         p0k_rowstats (the (mean, rstd) feed of the rms / lnmod prologues)
 *   defaultTune / DEFAULT_TILE src/core/tune.js:30-36, gemm.js:22  p0k_select_tile
 *   (timing: performance.now around gpu.done(), bench/bench.js:69-78)  p0k_event_* (HIP events on the context's stream)
 *
 * Conventions
 *   - Buffers are device pointers returned by p0k_alloc. Every operand is given as (buffer, offset, size); offsets of
 *     x / w / y are in BYTES, offsets of the fp32 vectors (ev, stats, pv, bv, rope) are in FLOATS (stats: in ROWS of
 *     two floats), exactly as in the reference's argument objects.
 *   - Sizes are the bytes the caller owns from `buf` onwards (the whole buffer, like the reference's `buf._pf`). They are
 *     required: p0k_gemm refuses any call whose reads or writes would leave them (the reference binds whole buffers and
 *     relies on WebGPU's robust access; a HIP kernel has no such guard).
 *   - Every call returns P0K_OK (0) or an error code; p0k_last_error() gives the message. Errors in the arguments are
 *     found on the host before anything is launched, and nothing is launched then.
 *   - All work of one context runs in order on one HIP stream (default priority). p0k_gemm only enqueues.
 */
#ifndef P0K_H
#define P0K_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 4: the measurement probes moved to the benchmark's own library; p0k_ctx_stream, p0k_gemm_plan,
 *    p0k_ctx_workspace_stats added */
#define P0K_ABI_VERSION 4

/* ---- status codes */
enum {
  P0K_OK = 0,
  P0K_E_ARG = 1,          /* bad argument (the reference throws Error(...) for these) */
  P0K_E_HIP = 2,          /* a HIP runtime error (the reference's GpuError / device lost) */
  P0K_E_NOMEM = 3,        /* device allocation failed */
  P0K_E_UNSUPPORTED = 4,  /* a combination this build does not implement */
};

/* ---- weight encodings (docs/FORMAT.md of the reference; gemm.js:269-271 maps the strings) */
enum { P0K_ENC_Q4G32A_T64 = 1, P0K_ENC_Q8G64S_T64 = 2, P0K_ENC_F16 = 3 };
/* ---- prologues: how X is read (gemm.js:60-95); conv / conv3 come from args.conv.kind in the reference */
enum { P0K_X_F16 = 0, P0K_X_LNMOD = 1, P0K_X_RMS = 2, P0K_X_CONV = 3, P0K_X_CONV3 = 4 };
/* ---- epilogues: how Y is written (gemm.js:191-254) */
enum { P0K_EPI_F16 = 0, P0K_EPI_F32 = 1, P0K_EPI_RESADD = 2, P0K_EPI_SWIGLU = 3, P0K_EPI_HEADS = 4, P0K_EPI_BIAS = 5,
       P0K_EPI_ONORMGATE = 6 };
enum { P0K_ACT_SILU = 0, P0K_ACT_GELU = 1 };                 /* args.act */
enum { P0K_ROPE_INTERLEAVED = 0, P0K_ROPE_HALF = 1 };        /* args.heads.ropeMode: default / 'half' */
/* args.acc. The reference's 'f16' mode (fp16 partial sums within each 32-k step, gemm.js:176-187) is a WebGPU ALU
 * speed trick; fp16 MFMA accumulates in fp32 at the same rate, so both modes compute with fp32 accumulation here, which
 * is at least as accurate as either reference mode and stays inside the tolerance both are tested against. */
enum { P0K_ACC_F32 = 0, P0K_ACC_F16 = 1 };

typedef struct p0k_ctx p0k_ctx;

/* One GEMM call: Y[m, n] = epilogue( sum_k X'[m, k] * W[n, k] ), X' = prologue(X) rounded to fp16, W dequantised to fp16.
 * Field names follow GemmArgs (types/index.d.ts:128-150) and the uniform P (gemm.js:39-41). Zero-initialise the struct
 * (all-zero = the reference's defaults) and set struct_size = sizeof(p0k_gemm_args). */
typedef struct p0k_gemm_args {
  uint32_t struct_size;
  /* w: {enc, buf, off, bytes, rows, cols, ld} */
  int32_t w_enc;
  const void *w_buf; uint64_t w_off, w_bytes;
  uint32_t w_rows, w_cols, w_ld;             /* rows = Nw, cols = Ktot; ld: f16 row stride in halves (0 = cols) */
  /* x: {buf, off, size, ld, k0, mode} */
  const void *x_buf; uint64_t x_off, x_size;
  uint32_t x_ld, x_k0;                       /* ld 0 = K */
  int32_t x_mode;                            /* P0K_X_F16 | LNMOD | RMS; CONV / CONV3 for args.conv */
  /* y: {buf, off, size, ld, n0} */
  void *y_buf; uint64_t y_off, y_size;
  uint32_t y_ld, y_n0;                       /* ld 0 = N */
  uint32_t M, N, K;
  int32_t epi, acc;
  uint32_t tile_bm, tile_bn;                 /* args.tile; 0 = choose (p0k_select_tile) */
  uint32_t wr0, wr1, wk0;
  /* fp32 vectors: (buf, off in floats, size in bytes from buf) */
  const float *ev_buf; uint32_t ev_off; uint64_t ev_size;          /* gate (resadd), bias (bias), norm weights (heads) */
  const float *st_buf; uint32_t st_off; uint64_t st_size;          /* stats: (mean, rstd) rows; off in rows */
  const float *pv_buf; uint32_t pv_off, pv_stride; uint64_t pv_size; /* prologue vectors: gamma / scale (+stride: shift) */
  const float *bv_buf; uint32_t bv_off, bv_up; uint64_t bv_size;   /* bias of resadd / swiglu (up at +bv_up) */
  const void *gt_buf; uint64_t gt_size;                            /* onormgate gate, fp16 [M][Ltot] */
  const float *rope_buf; uint64_t rope_size;                       /* heads: RP[row][64][cos, sin] */
  int32_t res, store, act;
  /* heads: {Ltot, Hq, Hkv, rowOff, eps, ropeMode} (eps 0 = 1e-6, as gemm.js:319) */
  uint32_t h_Ltot, h_Hq, h_Hkv, h_rowOff; float h_eps; int32_t h_rope_mode;
  /* conv: {Hi, Wi, Ci, Ho, Wo, stride, padT, padL, ks, up2, gn, pn} (stride 0 = 1, ks 0 = 1) */
  uint32_t c_Hi, c_Wi, c_Ci, c_Ho, c_Wo, c_stride, c_padT, c_padL, c_ks;
  int32_t c_up2, c_gn, c_pn;
} p0k_gemm_args;

/* rowstats (src/ops/misc.js:37-44): ST[(st_off + r) * 2 + {0, 1}] = (mean, rstd) of rows r of an fp32 [rows][ld] matrix,
 * columns [c0, c0 + cols); mode 0 = LayerNorm (mean, biased variance), 1 = RMSNorm (mean 0). */
typedef struct p0k_rowstats_args {
  uint32_t struct_size;
  const void *x_buf; uint64_t x_off, x_size;  /* x_off in bytes */
  uint32_t ld, c0, rows, cols;               /* ld 0 = cols */
  int32_t mode; float eps;
  float *st_buf; uint32_t st_off; uint64_t st_size;
} p0k_rowstats_args;

/* pixstats (src/ops/video.js:301-321): R[ro + v] = 1 / sqrt(sum_c x[v][c]^2 / C + eps) for voxels v < V of an f16
 * [V][C] tensor (C % 4 == 0) - the per-voxel scale the conv3 `pn` prologue reads. eps 0 = the reference's 1e-8. */
typedef struct p0k_pixstats_args {
  uint32_t struct_size;
  const void *x_buf; uint64_t x_off, x_size;  /* x_off in bytes */
  uint32_t V, C; float eps;
  float *r_buf; uint32_t ro; uint64_t r_size;  /* ro in floats */
} p0k_pixstats_args;

/* GroupNorm(32) statistics (src/ops/misc.js:50-109) of an HWC f16 tensor x [pix][C], C a power of two in 32..512:
 *   partial rows (gnPartial): part[(wg_off + w) * 32 + g] = (n, mean, M2, 0) per 64-pixel chunk w and group g
 *   finalize (gnFinalize):    merge nwg rows -> ab[ab_off + c] = gamma[c] / sqrt(M2 / n + eps),
 *                             ab[ab_off + C + c] = beta[c] - mean * ab[ab_off + c]   (GN(x) = a x + b per channel)
 * gamma / beta are fp32 vectors in gb_buf at byte offsets g_off / b_off (the reference's gb.gOff / gb.bOff).
 * eps 0 = the reference's 1e-6. */
typedef struct p0k_gn_args {
  uint32_t struct_size;
  const void *x_buf; uint64_t x_off, x_size;
  uint32_t pix, C;
  float *part_buf; uint32_t wg_off, nwg; uint64_t part_size;   /* nwg: rows to merge (finalize); 0 = ceil(pix / 64) */
  const float *gb_buf; uint64_t g_off, b_off, gb_size;
  float *ab_buf; uint32_t ab_off; uint64_t ab_size;             /* ab_off in floats */
  float eps;
} p0k_gn_args;

/* attention(gpu, a) (src/ops/attention.js:168-201), head size 128: Q [Hq][Lq][128], K / V [Hkv][Lk][128] f16 (the
 * `heads` epilogue's layout), O [Lq][ldo] f16 with head h at column h * 128. mode 0: no mask; 1: key j visible to query
 * i iff j <= min(i, nvalid - 1); 2: j < nvalid. GQA: query head h reads kv head h / (Hq / Hkv). Zero fields take the
 * reference's defaults: Lk = Lq, Hkv = Hq, nvalid = Lk, ldo = Hq * 128, scale = 1 / sqrt(128); cap > 0 soft-caps
 * the scores to cap * tanh(s / cap). Offsets and sizes in bytes; q / k / v offsets 16-byte aligned, o 8-byte. */
typedef struct p0k_attn_args {
  uint32_t struct_size;
  const void *q_buf; uint64_t q_off, q_size;
  const void *k_buf; uint64_t k_off, k_size;
  const void *v_buf; uint64_t v_off, v_size;
  void *o_buf; uint64_t o_off, o_size; uint32_t ldo;
  uint32_t Lq, Lk, Hq, Hkv, mode, nvalid;
  float scale, cap;
} p0k_attn_args;

typedef struct p0k_tile { uint32_t bm, bn; int32_t kernel; } /* kernel: 0 = MFMA GEMM (register-staged), 1 = GEMV (q4, M <= 4), 2 = MFMA GEMV (M <= 16), 3 = MFMA GEMM (load-to-LDS),
   4 = short-call GEMV (q4, q8 or f16, M <= 4, 16-row items) */
  p0k_tile;

typedef struct p0k_pool_stats {
  uint64_t alive, peak, pooled, high_water, max_buf;
  uint64_t creates, reuses, evictions, live_buffers, pooled_buffers;
} p0k_pool_stats;

typedef struct p0k_device_info {
  char name[64]; char arch[64];
  int32_t cus, xcds_hint; uint64_t hbm_bytes; int32_t clock_khz, mem_clock_khz, mem_bus_width;
} p0k_device_info;

/* ---- library */
int p0k_abi_version(void);
const char *p0k_last_error(void);            /* message of the last failed call on this thread */

/* ---- context (createGpu) */
int p0k_ctx_create(int device, p0k_ctx **out);
void p0k_ctx_destroy(p0k_ctx *ctx);
int p0k_device_info_get(p0k_ctx *ctx, p0k_device_info *out);
/* Kernel choice reads the device's CU count and the P0K_* tuning switches of the environment (P0K_MFMA_TILE,
 * P0K_MFMA_KERNEL, P0K_DMA_TAIL, P0K_GEMV_MF, P0K_GEMV_MQ4, P0K_GEMV_SLICES, P0K_ATTN_BQ) once, when the context is created;
 * p0k_ctx_reload_env reads the switches again (no counterpart in the reference, whose tuning is gpu.tune,
 * src/core/tune.js:30-36). p0k_ctx_cus: the CU count the context plans for. */
int p0k_ctx_reload_env(p0k_ctx *ctx);
int p0k_ctx_cus(p0k_ctx *ctx);
/* The context's HIP stream (a hipStream_t), for callers that enqueue their own work in order with the context's (no
 * counterpart in the reference, whose queue is gpu.device.queue, src/core/gpu.js:15-20). A caller may capture it into
 * a graph of its own: gemm calls enqueued under any capture keep the workspaces they use alive until the context goes. */
void *p0k_ctx_stream(p0k_ctx *ctx);
/* Device bytes held by the context's gemm workspaces (split-decode partials, the rms / lnmod X'), and how many
 * replaced workspaces it keeps because a graph captured after they were allocated may still address them. */
int p0k_ctx_workspace_stats(p0k_ctx *ctx, uint64_t *live_bytes, uint64_t *retired_buffers);

/* ---- buffers */
/* alloc / free return P0K_E_ARG while the context's stream is being captured into a graph (a clear or a hipFree
 * must not land in the graph). */
int p0k_alloc(p0k_ctx *ctx, uint64_t bytes, void **out);        /* zeroed; reuses a pooled buffer of the same rounded size */
int p0k_free(p0k_ctx *ctx, void *buf);                          /* back to the pool (or released) */
int p0k_drain_pool(p0k_ctx *ctx);
int p0k_pool_stats_get(p0k_ctx *ctx, p0k_pool_stats *out);
int p0k_upload(p0k_ctx *ctx, void *dst, uint64_t dst_off, const void *src, uint64_t n);
int p0k_download(p0k_ctx *ctx, const void *src, uint64_t src_off, void *dst, uint64_t n);
int p0k_copy(p0k_ctx *ctx, void *dst, uint64_t dst_off, const void *src, uint64_t src_off, uint64_t n);
int p0k_sync(p0k_ctx *ctx);

/* ---- the op */
int p0k_gemm_check(const p0k_gemm_args *a);                    /* validation only (no context, no GPU) */
int p0k_gemm(p0k_ctx *ctx, const p0k_gemm_args *a);            /* validate + enqueue; returns the status */
double p0k_gemm_flops(const p0k_gemm_args *a);                 /* 2*M*N*K, the reference's return value (gemm.js:326) */
/* p0k_gemm_noalloc: p0k_gemm that allocates nothing. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The
 * same kernels, with every workspace (split-decode partials and counters, the rms / lnmod / PixelNorm X', the conv3
 * zero block) taken from one static device array per GPU, set up when the first context on that GPU is created.
 * A call needing more than p0k_gemm_noalloc_scratch_bytes() (31.5 MiB: e.g. X' of M * K * 2 bytes) is refused with
 * P0K_E_ARG. The first context that calls it on a GPU holds that GPU's array until the context is destroyed, and calls
 * from any other context on the GPU are refused with P0K_E_ARG (their stream could overlap the holder's calls). Calls
 * in order on the holder's stream do not race; each call may overwrite what the previous one left in the array.
 * Results are the same bits as p0k_gemm's. */
int p0k_gemm_noalloc(p0k_ctx *ctx, const p0k_gemm_args *a);
uint64_t p0k_gemm_noalloc_scratch_bytes(void);
int p0k_select_tile(const p0k_gemm_args *a, p0k_tile *out);     /* the kernel and tile p0k_gemm would use on a
                                                                   256-CU device with the current environment */
int p0k_gemm_plan(p0k_ctx *ctx, const p0k_gemm_args *a, p0k_tile *out);   /* the kernel and tile p0k_gemm uses on
                                                                   this context (its CU count and tuning switches) */
int p0k_rowstats_check(const p0k_rowstats_args *a);
int p0k_rowstats(p0k_ctx *ctx, const p0k_rowstats_args *a);

/* attention(gpu, a) -> 4 Lq Lk 128 Hq   src/ops/attention.js:168 */
int p0k_attention_check(const p0k_attn_args *a);
int p0k_attention(p0k_ctx *ctx, const p0k_attn_args *a);
double p0k_attention_flops(const p0k_attn_args *a);

/* pixstats(gpu, a)               src/ops/video.js:317  */
int p0k_pixstats(p0k_ctx *ctx, const p0k_pixstats_args *a);
/* gnPartBytes(pix)               src/ops/misc.js:92    bytes of the partial rows of pix pixels */
uint64_t p0k_gn_part_bytes(uint32_t pix);
/* gnPartial(gpu, a) -> nwg       src/ops/misc.js:94    */
int p0k_gn_partial(p0k_ctx *ctx, const p0k_gn_args *a, uint32_t *nwg_out);
/* gnFinalize(gpu, a)             src/ops/misc.js:101   */
int p0k_gn_finalize(p0k_ctx *ctx, const p0k_gn_args *a);
/* groupnormStats(gpu, a)         src/ops/misc.js:106   partial rows of the whole tensor, then finalize */
int p0k_groupnorm_stats(p0k_ctx *ctx, const p0k_gn_args *a);

/* ---- weight encoders on the host CPU (src/convert/encode.js:56-98): fp32 [rows][K] -> FORMAT.md bytes.
 *      out holds p0k_tensor_bytes(enc, rows, K) bytes; deq (optional) receives the fp32 dequantised weights. */
uint64_t p0k_tensor_bytes(int enc, uint32_t rows, uint32_t cols);
int p0k_pack_q4(const float *W, uint32_t rows, uint32_t K, uint8_t *out, float *deq);
int p0k_pack_q8(const float *W, uint32_t rows, uint32_t K, uint8_t *out, float *deq);
int p0k_pack_f16(const float *W, uint64_t n, uint16_t *out);

/* ---- HIP graphs: capture the context's stream (e.g. a decode step's gemm calls), then replay it with one launch.
 *      (The reference batches dispatches into command buffers, src/core/gpu.js:203-257; a graph is the HIP form.)
 *      Between begin and end only enqueueing calls may be made (p0k_gemm, p0k_rowstats, p0k_copy). */
typedef struct p0k_graph p0k_graph;
int p0k_graph_begin(p0k_ctx *ctx);
int p0k_graph_end(p0k_ctx *ctx, p0k_graph **out);
int p0k_graph_launch(p0k_ctx *ctx, p0k_graph *g);
void p0k_graph_destroy(p0k_graph *g);

/* ---- timing on the context's stream */
typedef struct p0k_event p0k_event;
int p0k_event_create(p0k_ctx *ctx, p0k_event **out);
int p0k_event_record(p0k_ctx *ctx, p0k_event *ev);
int p0k_event_elapsed_ms(p0k_event *start, p0k_event *stop, float *ms);   /* waits for stop */
void p0k_event_destroy(p0k_event *ev);

#ifdef __cplusplus
}
#endif
#endif /* P0K_H */
