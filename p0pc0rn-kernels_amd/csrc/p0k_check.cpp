// p0k_check.cpp — host-side argument validation of `gemm` and `rowstats`, and the translation of p0k_gemm_args into
// the kernel Params. Pure host code: it never touches the GPU, so every error path is testable without one.
//
// The reference throws for: an unknown encoding (src/ops/gemm.js:271), K % 32 != 0 (:283), a bad tile (:31) and a
// missing binding (:313). Those messages are kept. The reference binds whole WebGPU buffers and relies on robust buffer
// access; a HIP kernel has none, so this build also refuses any call whose reads or writes leave the given buffer sizes,
// and any alignment the 128-bit loads cannot honour (the reference's vec4 views need the same alignments, gemm.js:43-46).
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "../../include/p0k.h"
#include "p0k_device.h"
#include "p0k_internal.h"
#include "p0k_launch.h"

namespace p0k {

static int fail(std::string *err, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
static int fail(std::string *err, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (err) *err = buf;
  return P0K_E_ARG;
}

static const char *epi_name(int e) {
  static const char *n[] = {"f16", "f32", "resadd", "swiglu", "heads", "bias", "onormgate"};
  return e >= 0 && e <= 6 ? n[e] : "?";
}

#define NEED(cond, ...) \
  do {                  \
    if (!(cond)) return fail(err, __VA_ARGS__); \
  } while (0)
#define FITS(what, need, have)                                                                                       \
  do {                                                                                                               \
    uint64_t n_ = (need), h_ = (have);                                                                               \
    if (n_ > h_)                                                                                                     \
      return fail(err, "gemm: %s needs %llu bytes from its offset, the buffer holds %llu", what, (unsigned long long)n_, \
                  (unsigned long long)h_);                                                                            \
  } while (0)

// size of [off, end) available in a (buf, off, size) operand
static uint64_t avail(uint64_t size, uint64_t off) { return size > off ? size - off : 0; }

Tuning tuning_from_env(unsigned cus) {
  Tuning t;
  t.cus = cus ? cus : 256;
  if (const char *ov = getenv("P0K_GEMV_MF")) t.gemv_mf = atoi(ov) != 0;
  if (const char *ov = getenv("P0K_GEMV_MQ4")) t.gemv_mq4 = atoi(ov) != 0;
  if (const char *ov = getenv("P0K_GEMV_SLICES")) t.gemv_slices = (unsigned)std::max(0, atoi(ov));
  if (const char *ov = getenv("P0K_GEMV_MX")) t.gemv_mx = (unsigned)std::max(0, atoi(ov));
  if (const char *ov = getenv("P0K_GEMV_NARROW")) t.gemv_narrow = atoi(ov) != 0;
  if (const char *ov = getenv("P0K_GEMV_SN")) t.gemv_sn = atoi(ov) != 0;
  if (const char *ov = getenv("P0K_MFMA_KERNEL")) t.mfma_reg = strcmp(ov, "reg") == 0;
  if (const char *ov = getenv("P0K_MFMA_TILE")) {
    unsigned tm = 0, tn = 0;
    if (sscanf(ov, "%ux%u", &tm, &tn) == 2 && (tm == 128 || tm == 256) && (tn == 128 || tn == 256)) {
      t.tile_m = tm;
      t.tile_n = tn;
    }
  }
  if (const char *ov = getenv("P0K_DMA_TAIL")) t.dma_tail = atoi(ov) != 0;
  if (const char *ov = getenv("P0K_ATTN_BQ")) {
    const int v = atoi(ov);
    if (v == 128 || v == 256) t.attn_bq = v;
  }
  return t;
}

// Where the short-call decode items are taken. q4: at most about one 16-row item per CU (one and a half at one row),
// one or two rows, K up to 8192. Measured per call against the planner's other choice (ring kernels, 64-column items or
// a K split), q4, K 4096 unless stated: plain N 2048 M 1 3.88 vs 6.07 us, M 2 5.35 vs 6.79; N 4096 M 1 4.45 vs 6.17,
// M 2 6.06 vs 6.89, M 4 7.92 vs 7.35; N 6144 M 1 6.02 vs 6.43, M 2 7.77 vs 7.08; N 14336 M 1 9.71 vs 7.98; N 4096
// K 8192 M 1 7.81 vs 9.98; K 14336 12.0 vs 11.9; SwiGLU out 4096 (8192 weight rows) M 1 7.91 vs 7.57. (A plain
// one-launch read of the same 10.5 MB as N 4096 K 4096 takes 4.3-4.5 us: the short calls are latency, not bytes.)
// q8 (against the matrix-core decode): every q8 call at one row, with up to 2 items per CU at two rows and 1 at 3..4
// rows, K up to 8192 (all that fits): plain N 4096 K 4096 M 1 / 2 / 4 5.21 / 6.67 / 8.57 vs 9.58 / 9.71 / 9.95 us;
// N 2048 4.44 / 5.91 / 7.68 vs 9.34 / 9.50 / 9.70; K 2048 4.12 / 4.76 / 5.88 vs 6.99 / 7.10 / 7.28; N 8192 M 1 / 2
// 7.48 / 9.68 vs 10.16 / 10.25 (M 4 13.17 vs 10.49); N 14336 M 1 11.93 vs 12.69 (M 2 15.13 vs 12.59); N 4096 K 8192
// M 1 / 2 9.47 / 11.31 vs 13.56 / 13.71; SwiGLU out 4096 M 1 / 2 7.64 / 9.66 vs 11.69 / 11.74, out 7168 M 1 12.15 vs
// 13.93, out 14336 (28672 weight rows, 121 MB) 20.79 vs 22.43; N 20480 / 28672 M 1 15.85 / 20.28 vs 20.90 / 22.43;
// N 6144 M 4 11.95 vs 10.29, N 10240 M 2 11.64 vs 10.71, N 28672 M 2 24.96 vs 22.57 (not taken).
// f16 (16-byte rows; against the matrix-core decode): every call with 1..4 rows and K up to 8192: N 4096 K 4096 M 1 / 2
// / 4 6.97 / 7.96 / 9.42 vs 14.21 / 14.31 / 14.38 us; N 2048 5.28 / 6.20 / 7.57 vs 14.43 / 15.26 / 15.34; N 8192
// 11.55 / 12.69 / 15.05 vs 29.63 / 29.71 / 29.94; N 14336 K 2048 10.89 / 11.21 / 12.68 vs 21.99 / 22.10 / 22.35; N 14336
// K 4096 19.09 / 20.30 / 24.94 vs 28.35 / 28.57 / 28.95; N 4096 K 8192 12.87 / 14.14 / 16.78 vs 26.92 / 27.16 / 27.37;
// SwiGLU out 7168 19.43 / 20.46 / 25.33 vs 30.26 / 29.54 / 29.75.
static bool sn_rule(int we, uint32_t N, uint32_t K, uint32_t M, unsigned cus) {
  const uint64_t items = (N + 15u) / 16u;
  if (we == P0K_ENC_F16) return true;
  if (we == P0K_ENC_Q8G64S_T64)
    return K <= 8192u && (M == 1 || (M == 2 ? items <= (uint64_t)cus * 2u : items <= cus));
  return M <= 2 && K <= 8192u && items * 2u <= (uint64_t)cus * (M == 1 ? 3u : 2u);
}

int prepare_gemm(const p0k_gemm_args *a, Params *out, Plan *plan, std::string *err, const Tuning &tune) {
  NEED(a != nullptr, "gemm: no arguments");
  NEED(a->struct_size == sizeof(p0k_gemm_args), "gemm: struct_size %u, this library expects %u (ABI %d)", a->struct_size,
       (unsigned)sizeof(p0k_gemm_args), P0K_ABI_VERSION);
  const int we = a->w_enc;
  NEED(we == P0K_ENC_Q4G32A_T64 || we == P0K_ENC_Q8G64S_T64 || we == P0K_ENC_F16, "gemm: unsupported weight encoding %d", we);
  const uint32_t M = a->M, N = a->N, K = a->K;
  NEED(K % 32 == 0, "gemm: K must be a multiple of 32");
  const int epi = a->epi, xm = a->x_mode;
  NEED(epi >= P0K_EPI_F16 && epi <= P0K_EPI_ONORMGATE, "gemm: unknown epilogue %d", epi);
  NEED(xm >= P0K_X_F16 && xm <= P0K_X_CONV3, "gemm: unknown x mode %d", xm);
  NEED(a->act == P0K_ACT_SILU || a->act == P0K_ACT_GELU, "gemm: unknown act %d", a->act);
  NEED(a->h_rope_mode == P0K_ROPE_INTERLEAVED || a->h_rope_mode == P0K_ROPE_HALF, "gemm: unknown ropeMode %d", a->h_rope_mode);
  NEED(a->acc == P0K_ACC_F32 || a->acc == P0K_ACC_F16, "gemm: unknown acc %d", a->acc);
  if (a->tile_bm || a->tile_bn) {                                      // gemm.js:31 (heads / onormgate force BN = 128)
    uint32_t bm = a->tile_bm, bn = (epi == P0K_EPI_HEADS || epi == P0K_EPI_ONORMGATE) ? 128 : a->tile_bn;
    NEED(bm && bn && bm % 32 == 0 && bn % 64 == 0 && (bn / 8) * (bm / 8) <= 256, "bad tile %ux%u", a->tile_bm, a->tile_bn);
  }
  const bool xf32 = xm == P0K_X_LNMOD || xm == P0K_X_RMS, conv = xm == P0K_X_CONV, conv3 = xm == P0K_X_CONV3;
  // ---- bindings the reference's kernel declares for this configuration (gemm.js:43-54, :313)
  char key[96];
  snprintf(key, sizeof key, "gemm.%d.%d.%s", we, xm, epi_name(epi));
  NEED(a->x_buf, "gemm: missing binding X for %s", key);
  NEED(a->w_buf, "gemm: missing binding W for %s", key);
  NEED(a->y_buf, "gemm: missing binding Y for %s", key);
  NEED(!(xf32 || (conv3 && a->c_pn)) || a->st_buf, "gemm: missing binding ST for %s", key);
  NEED(!(xf32 || (conv && a->c_gn)) || a->pv_buf, "gemm: missing binding PV for %s", key);
  NEED(!(epi == P0K_EPI_BIAS || epi == P0K_EPI_HEADS || epi == P0K_EPI_ONORMGATE) || a->ev_buf, "gemm: missing binding EV for %s", key);
  NEED(epi != P0K_EPI_ONORMGATE || a->gt_buf, "gemm: missing binding GT for %s", key);
  NEED(epi != P0K_EPI_HEADS || a->rope_buf, "gemm: missing binding RP for %s", key);

  Params p;
  memset(&p, 0, sizeof p);
  p.M = M; p.N = N; p.K = K;
  p.ldx = a->x_ld ? a->x_ld : K;
  p.kx0 = a->x_k0;
  p.wR0 = a->wr0; p.wR1 = a->wr1; p.wk0 = a->wk0;
  p.ldy = a->y_ld ? a->y_ld : N;
  p.ny0 = a->y_n0;
  p.rowOff = a->h_rowOff; p.Ltot = a->h_Ltot; p.Hq = a->h_Hq; p.Hkv = a->h_Hkv;
  p.eps = a->h_eps != 0.0f ? a->h_eps : 1e-6f;
  p.pvOff = a->pv_buf ? a->pv_off : 0; p.pvStride = a->pv_buf ? a->pv_stride : 0;
  p.evOff = a->ev_buf ? a->ev_off : 0; p.statOff = a->st_buf ? a->st_off : 0;
  p.Hi = a->c_Hi; p.Wi = a->c_Wi; p.Ci = a->c_Ci; p.Ho = a->c_Ho; p.Wo = a->c_Wo;
  p.stride = a->c_stride ? a->c_stride : 1; p.padT = a->c_padT; p.padL = a->c_padL; p.ks = a->c_ks ? a->c_ks : 1;
  p.Nw = a->w_rows;
  p.bvOff = a->bv_buf ? a->bv_off : 0; p.bvUp = a->bv_buf ? a->bv_up : 0;
  p.epi = epi;
  uint32_t f = 0;
  if (a->ev_buf && epi == P0K_EPI_RESADD) f |= F_GATE;
  if (a->bv_buf) f |= F_BIAS;
  if (a->store) f |= F_STORE;
  if (a->res) f |= F_RES;
  if (a->act == P0K_ACT_GELU) f |= F_GELU;
  if (a->h_rope_mode == P0K_ROPE_HALF) f |= F_ROPE_HALF;
  if (conv3 && a->c_pn) f |= F_PN;
  if (conv && a->c_gn) f |= F_GN;
  if (conv && a->c_up2) f |= F_UP2;

  // ---- weights
  const uint32_t Nw = a->w_rows, Kt = a->w_cols;
  NEED(Nw > 0 && Kt > 0, "gemm: w.rows and w.cols must be positive");
  uint64_t wbytes;
  if (we == P0K_ENC_Q4G32A_T64) {
    NEED(Nw % 64 == 0 && Kt % 32 == 0, "gemm: q4g32a.t64 needs rows %% 64 == 0 and cols %% 32 == 0");
    NEED(a->wk0 % 32 == 0, "gemm: wk0 must be a multiple of 32 for q4g32a.t64");
    p.wG = Kt / 32;
    wbytes = (uint64_t)(Nw / 64) * (Kt / 32) * 1280;
    NEED(a->w_off % 16 == 0, "gemm: w.off must be 16-byte aligned");
  } else if (we == P0K_ENC_Q8G64S_T64) {
    NEED(Nw % 64 == 0 && Kt % 64 == 0, "gemm: q8g64s.t64 needs rows %% 64 == 0 and cols %% 64 == 0");
    NEED(a->wk0 % 32 == 0, "gemm: wk0 must be a multiple of 32");
    p.wG = Kt / 64;
    wbytes = (uint64_t)(Nw / 64) * (Kt / 64) * 4224;
    NEED(a->w_off % 16 == 0, "gemm: w.off must be 16-byte aligned");
  } else {
    p.wG = a->w_ld ? a->w_ld : Kt;
    NEED(p.wG >= Kt, "gemm: w.ld (%u) < w.cols (%u)", p.wG, Kt);
    NEED(p.wG % 4 == 0 && a->wk0 % 4 == 0 && a->w_off % 8 == 0, "gemm: f16 weights need w.ld, wk0 multiples of 4 and w.off of 8 bytes");
    wbytes = ((uint64_t)(Nw - 1) * p.wG + Kt) * 2;
    if (p.wG % 8 == 0 && a->wk0 % 8 == 0 && a->w_off % 16 == 0) f |= F_WALIGN8;
  }
  FITS("w", wbytes, a->w_bytes);
  NEED((uint64_t)a->wk0 + K <= Kt, "gemm: wk0 + K (%llu) exceeds w.cols (%u)", (unsigned long long)a->wk0 + K, Kt);
  if (epi == P0K_EPI_SWIGLU) {
    NEED(N % 2 == 0, "gemm: swiglu needs an even N (gate and up columns interleave)");
    NEED((uint64_t)a->wr0 + N / 2 <= Nw && (uint64_t)a->wr1 + N / 2 <= Nw, "gemm: swiglu rows wr0/wr1 + N/2 exceed w.rows");
  }

  // ---- X
  const uint64_t xav = avail(a->x_size, 0);
  if (xm == P0K_X_F16) {
    NEED(p.ldx % 4 == 0 && p.kx0 % 4 == 0 && a->x_off % 8 == 0, "gemm: x.ld and x.k0 must be multiples of 4 (vec4 rows)");
    if (M) FITS("x", a->x_off + ((uint64_t)(M - 1) * p.ldx + p.kx0 + K) * 2, xav);
    if (p.ldx % 8 == 0 && p.kx0 % 8 == 0 && a->x_off % 16 == 0) f |= F_XALIGN8;
  } else if (xf32) {
    NEED(p.ldx % 4 == 0 && p.kx0 % 4 == 0 && a->x_off % 16 == 0, "gemm: fp32 x needs x.ld, x.k0 multiples of 4 and a 16-byte x.off");
    if (M) FITS("x", a->x_off + ((uint64_t)(M - 1) * p.ldx + p.kx0 + K) * 4, xav);
    NEED(p.pvOff % 4 == 0 && p.pvStride % 4 == 0, "gemm: pv.off and pv.stride must be multiples of 4 floats");
    FITS("stats", ((uint64_t)p.statOff + M) * 8, a->st_size);
    uint64_t pvn = (uint64_t)p.pvOff + (xm == P0K_X_LNMOD ? p.pvStride : 0) + p.kx0 + K;
    FITS("pv", pvn * 4, a->pv_size);
  } else {
    NEED(p.Ci > 0 && p.Ci % 32 == 0, "gemm: conv needs Ci %% 32 == 0 (one tap per 32-k step)");
    NEED(p.Hi && p.Wi && p.Ho && p.Wo, "gemm: conv needs Hi, Wi, Ho, Wo");
    NEED(a->x_off % 16 == 0, "gemm: conv x.off must be 16-byte aligned");
    if (conv) {
      NEED(K <= p.ks * p.ks * p.Ci, "gemm: conv K (%u) exceeds ks*ks*Ci", K);
      FITS("x", a->x_off + (uint64_t)p.Hi * p.Wi * p.Ci * 2, xav);
      if (a->c_gn) FITS("pv", ((uint64_t)p.pvOff + p.pvStride + p.Ci) * 4, a->pv_size);
      NEED(!a->c_gn || (p.pvOff % 4 == 0 && p.pvStride % 4 == 0), "gemm: pv.off and pv.stride must be multiples of 4 floats");
    } else {
      NEED(K <= 27 * p.Ci, "gemm: conv3 K (%u) exceeds 27*Ci", K);
      const uint32_t T = p.stride;
      uint64_t frames;
      if (M) {
        uint64_t otmax = (uint64_t)(M - 1) / ((uint64_t)p.Ho * p.Wo);
        int64_t lo = (int64_t)p.padT - 1, hi = (int64_t)otmax + p.padT + 1;
        lo = lo < 0 ? 0 : (lo > T - 1 ? T - 1 : lo);
        hi = hi < 0 ? 0 : (hi > T - 1 ? T - 1 : hi);
        if (p.ks > 1) {
          frames = p.ks;
        } else {
          NEED(lo >= (int64_t)p.padL, "gemm: conv3 reads clip frame %lld but the input buffer starts at frame padL=%u", (long long)lo, p.padL);
          frames = (uint64_t)(hi - p.padL + 1);
        }
        FITS("x", a->x_off + frames * p.Hi * p.Wi * p.Ci * 2, xav);
        p.nvox = frames * p.Hi * p.Wi < (1ull << 32) ? (uint32_t)(frames * p.Hi * p.Wi) : 0xffffffffu;
        if (a->c_pn) FITS("stats", frames * p.Hi * p.Wi * 4, a->st_size);
      }
    }
  }

  // ---- Y and the epilogue vectors
  const uint64_t yav = avail(a->y_size, 0);
  NEED(a->y_off % 4 == 0, "gemm: y.off must be a multiple of 4 bytes");
  if (M && N) {
    const uint64_t rowspan = (uint64_t)(M - 1) * p.ldy + p.ny0;
    switch (epi) {
    case P0K_EPI_F16: case P0K_EPI_BIAS:
      FITS("y", a->y_off + (rowspan + N) * 2, yav); break;
    case P0K_EPI_F32: case P0K_EPI_RESADD:
      FITS("y", a->y_off + (rowspan + N) * 4, yav); break;
    case P0K_EPI_SWIGLU:
      FITS("y", a->y_off + (rowspan + N / 2) * 2, yav); break;
    case P0K_EPI_ONORMGATE: {
      NEED(N % 128 == 0, "gemm: onormgate needs N %% 128 == 0 (one head per 128 columns)");
      FITS("y", a->y_off + (rowspan + N) * 2, yav);
      FITS("gt", ((uint64_t)(M - 1) * p.Ltot + p.ny0 + N) * 2, a->gt_size);
      FITS("ev", ((uint64_t)p.evOff + 128) * 4, a->ev_size);
      break;
    }
    case P0K_EPI_HEADS: {
      NEED(N % 128 == 0, "gemm: heads needs N %% 128 == 0 (one head per 128 columns)");
      uint64_t hd = N / 128 - 1;
      FITS("y", a->y_off + ((hd * p.Ltot + p.rowOff + M - 1) * 128 + 128) * 2, yav);
      FITS("rope", ((uint64_t)p.rowOff + M) * 128 * 4, a->rope_size);
      uint64_t nh = N / 128, evn = 0;
      if (nh > p.Hq && p.Hkv > 0) evn = 256;
      else if (p.Hq > 0) evn = 128;
      if (evn) FITS("ev", ((uint64_t)p.evOff + evn) * 4, a->ev_size);
      break;
    }
    }
    if (epi == P0K_EPI_BIAS || (epi == P0K_EPI_RESADD && a->ev_buf)) FITS("ev", ((uint64_t)p.evOff + N) * 4, a->ev_size);
    if (a->bv_buf && epi == P0K_EPI_RESADD) FITS("bv", ((uint64_t)p.bvOff + N) * 4, a->bv_size);
    if (a->bv_buf && epi == P0K_EPI_SWIGLU) {
      uint64_t e0 = (uint64_t)p.bvOff + N / 2, e1 = (uint64_t)p.bvOff + p.bvUp + N / 2;
      FITS("bv", (e0 > e1 ? e0 : e1) * 4, a->bv_size);
    }
  }
  p.flags = f;

  // ---- kernel choice: the decode GEMV for M <= 16 unless a convolution (whose K order must not depend on M); below,
  //      the ring kernels first, then the short-call items where sn_rule takes them (q4 short calls, q8 at one row and
  //      short grids, f16 at 1..4 rows)
  int kernel = K_MFMA;
  unsigned S = 0, KS = 0;
  bool mx = false, narrow = false;
  if (M <= (uint32_t)GEMV_MAX_M && (xm == P0K_X_F16 || xf32) && M > 0) {
    // the GEMV reads q8 in whole 64-k records and f16 rows with 16-byte loads only
    // and addresses the tensor with 32-bit offsets
    if ((we != P0K_ENC_Q8G64S_T64 || a->wk0 % 64 == 0) && (we != P0K_ENC_F16 || (f & F_WALIGN8)) &&
        wbytes < (1ull << 32)) {
      // one or two q4 rows: the VALU stream (exact dot products of fp32-dequantised weights; one 16-byte load covers
      // 16 whole code rows; at M = 2, 19-20 us vs 20-22 on the matrix cores for N 28672, K 4096); 3..16 rows, and q8 /
      // f16 at any M <= 16: the matrix cores (the VALU stream's work grows with M: 31 vs 22 us at M = 4; and for q8 /
      // f16 its per-lane loads read 16 of every 64 bytes per load: q8 2.8 vs 3.6 TB/s, f16 1.4 vs 3.7)
      bool mf = M >= 3 || we != P0K_ENC_Q4G32A_T64;
      if (tune.gemv_mf >= 0) mf = mf && tune.gemv_mf != 0;   // tuning: the VALU stream for M > 1
      // q4 with 2..4 rows (P0K_GEMV_MX): the one-row stream with its per-unit sums on the matrix cores (4x4x4 blocks,
      // each lane's own weight row as a B column): 14.6-15.2 us at M = 2..4 against 15.3 (dot products) and 16.1-16.3
      // (k_gemv_mq4); with 8 or 16 rows it is slower than k_gemv_mq4 (18.3 / 28.0 vs 16.8 / 17.9 us)
      mx = we == P0K_ENC_Q4G32A_T64 && M >= 2 && M <= tune.gemv_mx;
      if (mx) mf = false;
      gemv_split(p, we, tune.cus, mf, mx, &S, &KS);
      // q4 with up to 4 rows that the planner would split: 64-column items with 8 K-eighths each instead, no K split
      // (the split's store-acknowledge-count-load chain at the end costs about 3 us), when those items fill the GPU
      // (plain q4 N 14336, 112 tiles: 8.1 vs 9.7 us per call) or each one's stream is short (40 K bytes, at most
      // 256 KB: one item per CU then streams at about 43 GB/s, its ring's bytes in flight over the memory latency;
      // N 4096 / 6144 / 8192 with K 4096: 6.2 / 6.5 / 6.5 against 8.9 / 10.1 / 8.7 us split; N 4096 K 14336: 15.7
      // against 12.0, so long K keeps the split)
      // (the matrix-core decode kernels, 5..16 q4 rows and q8 / f16 weights, the same with items of one 64-row half)
      const uint32_t tiles128 = (N + 127) / 128;
      // (q8 / f16 take the filled-grid rule only: N 14336 with one row, q8 K 4096 19.6 against 21.5 us split (with
      // the earlier 8-byte q8 loads), f16
      // K 2048 26.5 against 27.5; with 4 q8 rows 20.1 against 21.8. Their short items are mixed: f16 items of 256 KB,
      // N 4096 K 2048, 18.8 against 12.7 us at one row (one item per CU, streaming at about 14 GB/s) but 20.0 against
      // 21.3 at 8 rows and N 6144; so they stay split)
      const uint32_t kq8 = gemv_unit_k(we, mf) * 8u;   // k of one unit in each K-eighth
      const bool fill = 2 * tiles128 >= tune.cus * 7u / 8u;
      // (q8 too, items up to 288 KB, with X streamed per unit: q8 N 4096 K 4096 10.7 -> 9.5 us, N 6144 17.0 -> 9.8,
      // N 4096 K 2048 9.95 -> 6.9; f16 items stream slowly one per CU, 15.3 -> 17.6 us at N 4096 K 2048)
      const bool short_k = (we == P0K_ENC_Q4G32A_T64 && (uint64_t)K * 40u <= 256u * 1024u) ||
                           (we == P0K_ENC_Q8G64S_T64 && (uint64_t)K * 66u <= 288u * 1024u);
      if (tune.gemv_narrow && S >= 2 && (mf || (we == P0K_ENC_Q4G32A_T64 && M <= 4)) && epi != P0K_EPI_HEADS &&
          epi != P0K_EPI_ONORMGATE && (fill || short_k) && K <= gemv_ks_max(M, we, mf, mx) && K % kq8 == 0) {
        narrow = true;
        S = 1;
        KS = K;
      }
      // tuning override of the slice count (P0K_GEMV_SLICES=n), honoured only when it keeps whole units per wave
      if (tune.gemv_slices) {
        narrow = false;
        unsigned s2 = tune.gemv_slices, quant = gemv_unit_k(we, mf) * 4u;
        if (K % (s2 * quant) == 0 && K / s2 <= gemv_ks_max(M, we, mf, mx)) { S = s2; KS = K / s2; }
      }
      if (S) kernel = mf ? K_GEMV_MF : K_GEMV;
      // short calls (q4, q8, or f16 with 16-byte rows; up to 4 rows, element-wise epilogues): 16-row items, no K split, every load of an item
      // in flight at once (sn_rule above)
      const uint32_t snuk = we == P0K_ENC_Q4G32A_T64 ? 32u : 64u, snwk = we == P0K_ENC_F16 ? 8u : snuk;
      const bool sn_ok = (we != P0K_ENC_F16 || (f & F_WALIGN8)) && M <= 4 && epi != P0K_EPI_HEADS &&
                         epi != P0K_EPI_ONORMGATE && K % snuk == 0 && K <= gemv_sn_kmax(we) && a->wk0 % snwk == 0 &&
                         gemv_sn_lds(we, M <= 2 ? M : 4, K) <= 64u * 1024u;
      if (sn_ok && (tune.gemv_sn == 1 || (tune.gemv_sn < 0 && sn_rule(we, N, K, M, tune.cus)))) {
        kernel = K_GEMV_SN;
        S = 1;
        KS = K;
        narrow = false;
      }
    }
  }
  if (out) *out = p;
  if (plan) {
    plan->kernel = kernel; plan->we = we; plan->xm = xm; plan->bm = 16; plan->bn = kernel == K_GEMV_SN ? 16 : narrow ? 64 : 128; plan->mx = mx; plan->narrow = narrow;
    // the load-to-LDS kernel where it applies (P0K_MFMA_KERNEL=reg keeps the register-staged one, for tests)
    if (kernel == K_MFMA && gemm_dma_ok(p, we, xm, wbytes) && !tune.mfma_reg) kernel = plan->kernel = K_MFMA_DMA;
    if (kernel == K_MFMA_DMA) dma_tile(M, N, we, xm == P0K_X_CONV3 ? X_CONV3 : X_F16, tune.cus, &plan->bm, &plan->bn);
    if (kernel == K_MFMA) mfma_tile(M, N, tune.cus, &plan->bm, &plan->bn);
    if ((kernel == K_MFMA || kernel == K_MFMA_DMA) && tune.tile_m) {
      // tuning / test override of the tile (P0K_MFMA_TILE=256x128); results do not depend on it
      plan->bm = tune.tile_m;
      plan->bn = tune.tile_n;
    }
    plan->S = S; plan->KS = KS;
  }
  return P0K_OK;
}

int prepare_rowstats(const p0k_rowstats_args *a, std::string *err) {
  NEED(a != nullptr, "rowstats: no arguments");
  NEED(a->struct_size == sizeof(p0k_rowstats_args), "rowstats: struct_size %u, this library expects %u", a->struct_size,
       (unsigned)sizeof(p0k_rowstats_args));
  NEED(a->x_buf && a->st_buf, "rowstats: missing x or st buffer");
  NEED(a->mode == 0 || a->mode == 1, "rowstats: mode must be 0 (ln) or 1 (rms)");
  NEED(a->cols > 0, "rowstats: cols must be positive");
  NEED(a->x_off % 4 == 0, "rowstats: x.off must be a multiple of 4 bytes");
  uint32_t ld = a->ld ? a->ld : a->cols;
  if (a->rows) {
    uint64_t need = a->x_off + ((uint64_t)(a->rows - 1) * ld + a->c0 + a->cols) * 4;
    if (need > a->x_size) return fail(err, "rowstats: x needs %llu bytes, the buffer holds %llu", (unsigned long long)need, (unsigned long long)a->x_size);
    uint64_t sneed = ((uint64_t)a->st_off + a->rows) * 8;
    if (sneed > a->st_size) return fail(err, "rowstats: st needs %llu bytes, the buffer holds %llu", (unsigned long long)sneed, (unsigned long long)a->st_size);
  }
  return P0K_OK;
}

int prepare_attention(const p0k_attn_args *a, AttnParams *out, std::string *err) {
  NEED(a != nullptr, "attention: no arguments");
  NEED(a->struct_size == sizeof(p0k_attn_args), "attention: struct_size %u, this library expects %u", a->struct_size,
       (unsigned)sizeof(p0k_attn_args));
  NEED(a->q_buf && a->k_buf && a->v_buf && a->o_buf, "attention: missing q, k, v or o buffer");
  const uint32_t Lq = a->Lq, Lk = a->Lk ? a->Lk : a->Lq, Hq = a->Hq, Hkv = a->Hkv ? a->Hkv : a->Hq;
  const uint32_t nvalid = a->nvalid ? a->nvalid : Lk, ldo = a->ldo ? a->ldo : Hq * 128;
  NEED(Lq > 0 && Lk > 0 && Hq > 0, "attention: Lq, Lk and Hq must be positive");
  NEED(Hq % Hkv == 0, "attention: Hq %u is not a multiple of Hkv %u", Hq, Hkv);
  NEED(a->mode <= 2, "attention: mode must be 0, 1 or 2");
  NEED(nvalid <= Lk || a->mode == 0, "attention: nvalid %u exceeds Lk %u", nvalid, Lk);
  NEED(a->q_off % 16 == 0 && a->k_off % 16 == 0 && a->v_off % 16 == 0, "attention: q / k / v offsets must be 16-byte aligned");
  NEED(a->o_off % 8 == 0 && ldo % 4 == 0 && ldo >= Hq * 128, "attention: o offset 8-byte aligned, ldo a multiple of 4 covering Hq * 128");
  FITS("q", a->q_off + (uint64_t)Hq * Lq * 256, a->q_size);
  FITS("k", a->k_off + (uint64_t)Hkv * Lk * 256, a->k_size);
  FITS("v", a->v_off + (uint64_t)Hkv * Lk * 256, a->v_size);
  FITS("o", a->o_off + ((uint64_t)(Lq - 1) * ldo + Hq * 128) * 2, a->o_size);
  if (out) {
    out->Q = (const uint16_t *)((const uint8_t *)a->q_buf + a->q_off);
    out->K = (const uint16_t *)((const uint8_t *)a->k_buf + a->k_off);
    out->V = (const uint16_t *)((const uint8_t *)a->v_buf + a->v_off);
    out->O = (uint16_t *)((uint8_t *)a->o_buf + a->o_off);
    out->Lq = Lq; out->Lk = Lk; out->ldo = ldo; out->Hq = Hq; out->Hkv = Hkv; out->mode = a->mode; out->nvalid = nvalid;
    out->scale = a->scale != 0.0f ? a->scale : 0.08838834764831845f;   // 1 / sqrt(128)
    out->cap = a->cap;
  }
  return P0K_OK;
}

int prepare_pixstats(const p0k_pixstats_args *a, std::string *err) {
  NEED(a != nullptr, "pixstats: no arguments");
  NEED(a->struct_size == sizeof(p0k_pixstats_args), "pixstats: struct_size %u, this library expects %u", a->struct_size,
       (unsigned)sizeof(p0k_pixstats_args));
  NEED(a->x_buf && a->r_buf, "pixstats: missing x or r buffer");
  NEED(a->C > 0 && a->C % 4 == 0, "pixstats: C must be a positive multiple of 4");
  NEED(a->x_off % 2 == 0, "pixstats: x.off must be a multiple of 2 bytes");
  FITS("x", a->x_off + (uint64_t)a->V * a->C * 2, a->x_size);
  FITS("r", ((uint64_t)a->ro + a->V) * 4, a->r_size);
  return P0K_OK;
}

int prepare_gn(const p0k_gn_args *a, int what, std::string *err) {
  NEED(a != nullptr, "groupnorm: no arguments");
  NEED(a->struct_size == sizeof(p0k_gn_args), "groupnorm: struct_size %u, this library expects %u", a->struct_size,
       (unsigned)sizeof(p0k_gn_args));
  NEED(a->C >= 32 && a->C <= 512 && (a->C & (a->C - 1)) == 0, "groupnorm: C must be a power of two in 32..512");
  NEED(a->part_buf, "groupnorm: missing part buffer");
  if (what & 1) {
    NEED(a->x_buf, "groupnorm: missing x buffer");
    NEED(a->x_off % 2 == 0, "groupnorm: x.off must be a multiple of 2 bytes");
    FITS("x", a->x_off + (uint64_t)a->pix * a->C * 2, a->x_size);
    FITS("part", ((uint64_t)a->wg_off + (a->pix + 63) / 64) * 512, a->part_size);
  }
  if (what & 2) {
    NEED(a->gb_buf && a->ab_buf, "groupnorm: missing gb or ab buffer");
    NEED(a->g_off % 4 == 0 && a->b_off % 4 == 0, "groupnorm: gamma / beta offsets must be multiples of 4 bytes");
    const uint64_t nwg = a->nwg ? a->nwg : (a->pix + 63) / 64;
    FITS("part", nwg * 512, a->part_size);
    FITS("gb", (a->g_off > a->b_off ? a->g_off : a->b_off) + (uint64_t)a->C * 4, a->gb_size);
    FITS("ab", ((uint64_t)a->ab_off + 2ull * a->C) * 4, a->ab_size);
  }
  return P0K_OK;
}

}  // namespace p0k
