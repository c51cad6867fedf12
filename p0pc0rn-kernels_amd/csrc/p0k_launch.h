// p0k_launch.h — host-side launchers of the gfx950 kernels (one per kernel family), called by p0k_runtime.cpp.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace p0k {
struct Params;
constexpr int GEMV_MAX_M = 16;
// MFMA GEMM (any M): bm x bn tiles in {128, 256}^2, 512 threads; mfma_tile picks the tile for a shape
void mfma_tile(uint32_t M, uint32_t N, unsigned cus, unsigned *bm, unsigned *bn);
hipError_t launch_gemm_mfma(const Params &p, int we, int xm, unsigned bm, unsigned bn, hipStream_t s);
// MFMA GEMM with load-to-LDS operands (fp16 rows of X' in memory, or the conv3 gather of input voxels; q4 / q8 / f16
// weights decoded in registers). gemm_dma_ok: the call qualifies (prologue f16 with 16-byte rows, rms / lnmod
// materialised by launch_xprep into an M x K fp16 buffer, or conv3 with Ci % 64 == 0, its PixelNorm materialised by
// launch_xprep over the input voxels; K % 64 == 0). dma_tile picks the tile. xg: X_F16 (rows) or X_CONV3.
bool gemm_dma_ok(const Params &p, int we, int xm, uint64_t wbytes);
void dma_tile(uint32_t M, uint32_t N, int we, int xg, unsigned cus, unsigned *bm, unsigned *bn);
// the column split launch_gemm_dma makes for a mostly empty last round: columns [0, ncut) with the chosen tile, the
// rest with bm2 x bn2 (ncut == N: one launch)
void dma_tail(uint32_t M, uint32_t N, int we, unsigned bm, unsigned bn, unsigned cus, uint32_t *ncut, unsigned *bm2,
              unsigned *bn2);
// workgroups per CU of a tile for a grid of `tiles` (q4 256 x 128: 8 waves, one per CU, when the grid has at most one
// tile per CU; 4 waves, two per CU, otherwise): the planner scores tiles with it and the launcher picks the wave count
unsigned dma_wgs(int we, unsigned m, unsigned n, uint64_t tiles, unsigned cus);
hipError_t launch_xprep(const Params &p, int xm, uint16_t *xp, hipStream_t s);
// cus: the device's CU count; tail: allow the column split of dma_tail
hipError_t launch_gemm_dma(const Params &p, int we, int xg, unsigned bm, unsigned bn, unsigned cus, bool tail, hipStream_t s);
// decode GEMV (M <= 16, prologue f16 / rms / lnmod): items of 128 ws columns x K/S; S > 1 needs the workspace
// (part: S*M*N floats, cnt: one zeroed counter per 128-column tile). mf: the matrix-core variant (2 <= M <= 16);
// mq4: with q4 weights, its form without X' staging (k_gemv_mq4); mx: q4 at M = 2 takes the stream kernel's
// matrix-core form (4-row tile) instead of its dot-product form (q4 with 3..16 rows on the stream kernel always does);
// narrow: the stream kernel (q4, M <= 4, S = 1, element-wise epilogues) over items of 64 columns instead of 128
void gemv_split(const Params &p, int we, unsigned cus, bool mf, bool mx, unsigned *S, unsigned *KS);
unsigned gemv_ks_max(unsigned M, int we, bool mf, bool mx);   // longest K slice one item stages
unsigned gemv_unit_k(int we, bool mf);                      // k of one decode weight unit
hipError_t launch_gemv(const Params &p, int we, int xm, float *part, unsigned *cnt, unsigned S, unsigned KS, hipStream_t s,
                       bool mf, bool mq4, bool mx, bool narrow);
// short decode calls: q4 or q8, 1..4 rows, element-wise epilogues, K a multiple of the unit (32 / 64) and at most
// gemv_sn_kmax(we), LDS (gemv_sn_lds) at most 64 KB; items of 16 weight rows with no K split (ceil(N / 16) workgroups)
unsigned gemv_sn_kmax(int we);
unsigned gemv_sn_lds(int we, unsigned M, unsigned K);
hipError_t launch_gemv_sn(const Params &p, int we, int xm, hipStream_t s);
// rowstats (src/ops/misc.js:16-44)
hipError_t launch_rowstats(const void *x, unsigned ld, unsigned c0, unsigned rows, unsigned cols, int mode, float eps,
                           float *st, unsigned st_off, hipStream_t s);
// flash attention, head size 128 (src/ops/attention.js:168-201)
struct AttnParams {
  const uint16_t *Q, *K, *V;   // [Hq][Lq][128], [Hkv][Lk][128] f16
  uint16_t *O;                 // [Lq][ldo] f16, head h at column h * 128
  uint32_t Lq, Lk, ldo, Hq, Hkv, mode, nvalid;
  float scale, cap;            // natural-log scale; cap > 0: scores -> cap * tanh(scores / cap)
};
int attention_bq(uint32_t Lq, uint32_t Hq, int cus, int force);   // queries per workgroup (force: 128 / 256 or 0)
hipError_t launch_attention(const AttnParams &p, int cus, int force_bq, hipStream_t s);
// pixstats and GroupNorm statistics (src/ops/video.js:301-321, src/ops/misc.js:50-109)
hipError_t launch_pixstats(const void *x, uint32_t V, uint32_t C, float eps, float *r, hipStream_t s);
hipError_t launch_gn_partial(const void *x, uint32_t pix, uint32_t C, float *part, uint32_t wg_off, hipStream_t s);
hipError_t launch_gn_finalize(const float *part, uint32_t nwg, uint32_t C, float eps, const float *gamma,
                              const float *beta, float *ab, hipStream_t s);
}  // namespace p0k
