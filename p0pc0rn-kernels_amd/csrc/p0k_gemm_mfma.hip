// p0k_gemm_mfma.hip — the prefill / convolution path of `gemm` (src/ops/gemm.js:29-257) on gfx950 matrix cores.
//
// One workgroup (256 threads = 4 waves of 64) computes a 128 x 128 output tile; each wave a 64 x 64 quarter with
// v_mfma_f32_32x32x16_f16 (fp16 in, fp32 accumulate). Per 32-k step:
//   global -> registers : X rows (8 halfs / thread-chunk) and the weight codes (128-bit loads of the FORMAT.md records)
//   registers -> LDS    : the prologue (rms / lnmod / conv / conv3 address maths, PixelNorm, GroupNorm) or the
//                         q4 / q8 dequantisation, as fp16, in the pair order of the encoding (p0k_device.h)
//   LDS -> MFMA         : 2 x 16-k sub-steps, 2 x 2 32x32 blocks per wave
// The global loads for step k+1 are issued before the MFMAs of step k, so HBM latency hides behind the matrix work.
// After the last step the fp32 tile goes through LDS once and the shared epilogue writes it (bias, residual, GLU,
// heads, ...). The K order of every output element is the same whatever rows a call covers (no split-K, no
// M-dependent choice), so a time-chunked or ring-buffered conv3 call is bit-identical to the whole-clip call.
#include "p0k_device.h"
#include "p0k_launch.h"

namespace p0k {

constexpr int BM = 128, BN = 128, BK = 32, BKP = 40;   // LDS rows padded to 80 bytes
constexpr int NT = 256;
constexpr int SMEM_AB = (BM + BN) * BKP * 2;           // 20 KB
constexpr int LDC = BN + 4;
constexpr int SMEM_C = BM * LDC * 4;                   // 66 KB
constexpr int SMEM = SMEM_C > SMEM_AB ? SMEM_C : SMEM_AB;

// Tile order: consecutive workgroups go to different XCDs (round-robin), so the linear id is first regrouped per XCD,
// then walked in bands of 8 M-tiles so the workgroups resident on one XCD share X rows and weight columns in its L2.
__device__ __forceinline__ void tile_of(const Params &p, uint32_t bid, uint32_t &mt, uint32_t &nt) {
  const uint32_t total = p.tilesM * p.tilesN;
  uint32_t t = bid;
  if ((total & 7u) == 0u) t = (bid & 7u) * (total >> 3) + (bid >> 3);
  const uint32_t band = 8u;
  uint32_t per = band * p.tilesN, g = t / per, first = g * band;
  uint32_t rows = p.tilesM - first < band ? p.tilesM - first : band;
  uint32_t in = t - g * per;
  mt = first + in % rows;
  nt = in / rows;
}

template <int WE>
struct BRegs;
template <>
struct BRegs<W_Q4> { u32x2 code; uint32_t sm; };
template <>
struct BRegs<W_Q8> { u32x4 code; uint32_t s; };
template <>
struct BRegs<W_F16> { u32x4 v[2]; };

template <int WE, int XM>
__global__ __launch_bounds__(NT, 2) void k_gemm_mfma(Params p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];
  f16 *sA = (f16 *)smem, *sB = sA + BM * BKP;
  float *sC = (float *)smem;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t mt, nt;
  tile_of(p, blockIdx.x, mt, nt);
  const uint32_t mB = mt * BM, nB = nt * BN;

  // ---- A (X') chunks: rows tid/4 and tid/4 + 64, k offset 8*(tid&3) inside the step
  const int akc = tid & 3;
  int arow[2] = {tid >> 2, (tid >> 2) + 64};
  uint32_t am[2];
  RowCtx rc[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    uint32_t m = mB + arow[i];
    am[i] = m < p.M ? m : p.M - 1u;
    rc[i] = row_ctx<XM>(p, am[i]);
  }
  // ---- B (weights): q4 / q8: row tid/2, half (tid&1) of the 32-k step; f16: two 16-byte chunks
  const int brow = tid >> 1, bh = tid & 1;
  const uint32_t wr = wrow(p, nB + brow);
  uint32_t wr16[2];
  if constexpr (WE == W_F16) {
    wr16[0] = wrow(p, nB + (tid >> 2));
    wr16[1] = wrow(p, nB + (tid >> 2) + 64);
  }

  u32x4 ar[2];
  BRegs<WE> br;
  auto load = [&](uint32_t k0) {
#pragma unroll
    for (int i = 0; i < 2; i++) ar[i] = xload8<XM>(p, am[i], rc[i], k0 + 8 * akc);
    const uint32_t kc = p.wk0 + k0;
    if constexpr (WE == W_Q4) {
      const uint8_t *rec = p.W + ((size_t)(wr >> 6) * p.wG + (kc >> 5)) * 1280u;
      br.code = *(const u32x2 *)(rec + (wr & 63u) * 16u + bh * 8u);
      br.sm = *(const uint32_t *)(rec + 1024u + (wr & 63u) * 4u);
    } else if constexpr (WE == W_Q8) {
      const uint8_t *rec = p.W + ((size_t)(wr >> 6) * p.wG + (kc >> 6)) * 4224u;
      br.code = *(const u32x4 *)(rec + (wr & 63u) * 64u + ((kc >> 5) & 1u) * 32u + bh * 16u);
      br.s = *(const uint32_t *)(rec + 4096u + (wr & 62u) * 2u);
    } else {
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const uint8_t *src = p.W + ((size_t)wr16[i] * p.wG + kc + 8 * akc) * 2;
        if (p.flags & F_WALIGN8) {
          br.v[i] = *(const u32x4 *)src;
        } else {
          u32x2 lo = *(const u32x2 *)src, hi = *(const u32x2 *)(src + 8);
          br.v[i] = (u32x4){lo.x, lo.y, hi.x, hi.y};
        }
      }
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < 2; i++) *(u32x4 *)(sA + arow[i] * BKP + 8 * akc) = xperm<WE>(ar[i]);
    if constexpr (WE == W_Q4) {
      bool fast = q4_fast_ok(br.sm);
      f16x2 o0[4], o1[4];
      dq_q4_word(br.code.x, br.sm, fast, o0);
      dq_q4_word(br.code.y, br.sm, fast, o1);
      u32x4 *dst = (u32x4 *)(sB + brow * BKP + 16 * bh);
      dst[0] = (u32x4){as_u(o0[0]), as_u(o0[1]), as_u(o0[2]), as_u(o0[3])};
      dst[1] = (u32x4){as_u(o1[0]), as_u(o1[1]), as_u(o1[2]), as_u(o1[3])};
    } else if constexpr (WE == W_Q8) {
      uint32_t sh = (wr & 1u) ? (br.s >> 16) : (br.s & 0xffffu);
      f16x2 s2 = as_h2(sh | (sh << 16));
      f16x2 o[8];
      dq_q8_word(br.code.x, s2, o + 0);
      dq_q8_word(br.code.y, s2, o + 2);
      dq_q8_word(br.code.z, s2, o + 4);
      dq_q8_word(br.code.w, s2, o + 6);
      u32x4 *dst = (u32x4 *)(sB + brow * BKP + 16 * bh);
      dst[0] = (u32x4){as_u(o[0]), as_u(o[1]), as_u(o[2]), as_u(o[3])};
      dst[1] = (u32x4){as_u(o[4]), as_u(o[5]), as_u(o[6]), as_u(o[7])};
    } else {
#pragma unroll
      for (int i = 0; i < 2; i++) *(u32x4 *)(sB + ((tid >> 2) + 64 * i) * BKP + 8 * akc) = br.v[i];
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = (f32x16){};

  const int wm = wave >> 1, wn = wave & 1, l32 = lane & 31, kq = (lane >> 5) * 8;
  const uint32_t nk = p.K / BK;
  if (nk) load(0);
  for (uint32_t kt = 0; kt < nk; kt++) {
    store();
    __syncthreads();
    if (kt + 1 < nk) load((kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK; ks += 16) {
      f16x8 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; i++) a[i] = *(const f16x8 *)(sA + (wm * 64 + i * 32 + l32) * BKP + ks + kq);
#pragma unroll
      for (int j = 0; j < 2; j++) b[j] = *(const f16x8 *)(sB + (wn * 64 + j * 32 + l32) * BKP + ks + kq);
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  // ---- accumulators -> LDS tile (32x32 block layout: lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4, column l%32)
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        int row = wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        int col = wn * 64 + j * 32 + l32;
        sC[row * LDC + col] = acc[i][j][r];
      }
  __syncthreads();
  epilogue<NT>(p, sC, LDC, BM, mB, nB, tid);
}

template <int WE, int XM>
static hipError_t launch_one(const Params &p, hipStream_t s) {
  Params q = p;
  q.tilesM = (p.M + BM - 1) / BM;
  q.tilesN = (p.N + BN - 1) / BN;
  dim3 grid(q.tilesM * q.tilesN);
  hipLaunchKernelGGL((k_gemm_mfma<WE, XM>), grid, dim3(NT), 0, s, q);
  return hipGetLastError();
}

template <int WE>
static hipError_t launch_x(const Params &p, int xm, hipStream_t s) {
  switch (xm) {
  case X_F16: return launch_one<WE, X_F16>(p, s);
  case X_LNMOD: return launch_one<WE, X_LNMOD>(p, s);
  case X_RMS: return launch_one<WE, X_RMS>(p, s);
  case X_CONV: return launch_one<WE, X_CONV>(p, s);
  case X_CONV3: return launch_one<WE, X_CONV3>(p, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemm_mfma(const Params &p, int we, int xm, hipStream_t s) {
  switch (we) {
  case W_Q4: return launch_x<W_Q4>(p, xm, s);
  case W_Q8: return launch_x<W_Q8>(p, xm, s);
  case W_F16: return launch_x<W_F16>(p, xm, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace p0k
