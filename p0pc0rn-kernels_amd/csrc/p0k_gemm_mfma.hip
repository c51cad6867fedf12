// p0k_gemm_mfma.hip — the prefill / convolution path of `gemm` (src/ops/gemm.js:29-257) on gfx950 matrix cores.
//
// One workgroup (256 threads = 4 waves of 64) computes a TBM x TBN output tile, TBM, TBN in {128, 256}; the waves
// form a 2 x 2 grid, each owning a (TBM/2) x (TBN/2) block of 32x32 v_mfma_f32_32x32x16_f16 tiles (fp16 in, fp32
// accumulate; a 128 x 128 wave block keeps its 256 accumulators in AGPRs). Per 32-k step:
//   global -> registers : X rows (8 halfs per chunk) and the weight codes (the FORMAT.md records, read in place)
//   registers -> LDS    : the prologue (rms / lnmod / conv / conv3 address maths, PixelNorm, GroupNorm) or the
//                         q4 / q8 dequantisation, as fp16 in the pair order of the encoding (p0k_device.h)
//   LDS -> MFMA         : 2 x 16-k sub-steps
// LDS rows are 64 bytes (four 16-byte chunks of 8 k) with the chunk index XORed by bits 2-3 of the row: the 16-byte
// MFMA operand reads (16 lanes = 16 rows, one chunk) and the staging writes (4 rows x 4 chunks) both hit 64 distinct
// banks. LDS holds two stages and the registers two steps of loads: the loads for step k+2 are issued before the MFMAs
// of step k, and step k+1 (loaded during step k-1) is written to the other stage after them, so each step needs one
// barrier and L2 / MALL / HBM latency hides behind two steps of matrix work. Large tiles keep
// the dequant and prologue work per MFMA low (each X' element is produced once per TBN columns, each weight once per
// TBM rows) and the LDS read traffic per MFMA low (a wave reads TBM/2 + TBN/2 operand rows per TBM*TBN/4 outputs).
// After the last step the fp32 accumulators go through LDS in 128 x 128 quadrants, and the shared epilogue writes
// them (bias, residual, GLU, heads, ...). The K order of every output element is the same whatever tile or rows a
// call covers (no split-K), so a time-chunked or ring-buffered conv3 call is bit-identical to the whole-clip call.
#include "p0k_device.h"
#include "p0k_launch.h"

namespace p0k {

constexpr int BK = 32;            // k per step; an LDS row holds BK halfs = 64 bytes = 4 chunks
constexpr int NT = 256;
constexpr int LDC = 128 + 4;

template <int TBM, int TBN>
struct Tile {
  static constexpr int STAGE = (TBM + TBN) * BK;                   // halfs per LDS stage
  static constexpr int SMEM_AB = 2 * STAGE * 2;                    // bytes, two stages
  static constexpr int SMEM_C = 128 * LDC * 4;                     // one 128 x 128 quadrant of the fp32 tile
  static constexpr int SMEM = SMEM_C > SMEM_AB ? SMEM_C : SMEM_AB;
  static constexpr int WTM = TBM / 2, WTN = TBN / 2;               // per-wave block
  static constexpr int BI = WTM / 32, BJ = WTN / 32;               // 32x32 MFMA tiles per wave
  static constexpr int ACH = TBM * 4 / NT;                         // X chunks (8 k) per thread per step
  static constexpr int BCH = TBN * 4 / NT;                         // f16 weight chunks per thread per step
  static constexpr bool PF2 = TBM * TBN < 256 * 256;               // registers for loads two steps ahead
  static constexpr bool FRAG2 = TBM * TBN < 256 * 256;             // both sub-steps' MFMA operands read at once
};

// halfs offset of chunk c (8 k) of LDS row r
__device__ __forceinline__ int lds_off(int r, int c) { return r * BK + ((c ^ (r >> 2)) & 3) * 8; }

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

// Weight registers of one thread for one step.
//   q4: UW = 4 TBN / NT code words (8 k each) of one row + its (scale, min) word
//   q8: UW = 8 TBN / NT code words (4 k each) of one row + its scale word
//   f16: 4 TBN / NT chunks of 8 halfs
template <int WE, int TBN>
struct BRegs;
template <int TBN>
struct BRegs<W_Q4, TBN> { uint32_t code[TBN * 4 / NT]; uint32_t sm; };
template <int TBN>
struct BRegs<W_Q8, TBN> { uint32_t code[TBN * 8 / NT]; uint32_t s; };
template <int TBN>
struct BRegs<W_F16, TBN> { u32x4 v[TBN * 4 / NT]; };

// AL: the f16 operands (X rows for the f16 prologue, f16 weight rows) allow 16-byte loads
template <int WE, int XM, int TBM, int TBN, bool AL>
__global__ __launch_bounds__(NT, (TBM * TBN >= 256 * 256 ? 1 : 2))
__attribute__((amdgpu_waves_per_eu((TBM * TBN >= 256 * 256 ? 1 : 2), (TBM * TBN >= 256 * 256 ? 1 : 2)))) void k_gemm_mfma(Params p) {
  using T = Tile<TBM, TBN>;
  constexpr int UW = WE == W_Q4 ? TBN * 4 / NT : (WE == W_Q8 ? TBN * 8 / NT : 0);
  constexpr int TPR = WE == W_Q4 ? 4 / UW : (WE == W_Q8 ? 8 / UW : 4);   // threads per weight row
  __shared__ __attribute__((aligned(16))) uint8_t smem[T::SMEM];
  f16 *const s0 = (f16 *)smem;
  float *sC = (float *)smem;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t mt, nt;
  tile_of(p, blockIdx.x, mt, nt);
  const uint32_t mB = mt * TBM, nB = nt * TBN;

  // ---- X' chunks: rows tid/4 + 64 c, chunk tid&3 of the step
  const int akc = tid & 3;
  uint32_t am[T::ACH];
  RowCtx rc[T::ACH];
#pragma unroll
  for (int c = 0; c < T::ACH; c++) {
    uint32_t m = mB + (tid >> 2) + (NT / 4) * c;
    am[c] = m < p.M ? m : p.M - 1u;
    rc[c] = row_ctx<XM>(p, am[c]);
  }
  // ---- weights
  const int brow = WE == W_F16 ? (tid >> 2) : tid / TPR;
  const int bw0 = WE == W_F16 ? 0 : (tid % TPR) * UW;
  uint32_t wr[WE == W_F16 ? T::BCH : 1];
  if constexpr (WE == W_F16) {
#pragma unroll
    for (int c = 0; c < T::BCH; c++) wr[c] = wrow(p, nB + (tid >> 2) + (NT / 4) * c);
  } else {
    wr[0] = wrow(p, nB + brow);
  }

  struct Regs {
    u32x4 ar[T::ACH];
    BRegs<WE, TBN> br;
  };
  auto load = [&](Regs &R, uint32_t k0) __attribute__((always_inline)) {
    u32x4 *ar = R.ar;
    BRegs<WE, TBN> &br = R.br;
#pragma unroll
    for (int c = 0; c < T::ACH; c++) ar[c] = xload8<XM, AL ? 1 : 0>(p, am[c], rc[c], k0 + 8 * akc);
    const uint32_t kc = p.wk0 + k0;
    if constexpr (WE == W_Q4) {
      const uint8_t *rec = p.W + ((size_t)(wr[0] >> 6) * p.wG + (kc >> 5)) * 1280u;
      const uint8_t *src = rec + (wr[0] & 63u) * 16u + bw0 * 4u;
      if constexpr (UW == 4) {
        u32x4 v = *(const u32x4 *)src;
        br.code[0] = v.x; br.code[1] = v.y; br.code[2] = v.z; br.code[3] = v.w;
      } else {
        u32x2 v = *(const u32x2 *)src;
        br.code[0] = v.x; br.code[1] = v.y;
      }
      br.sm = *(const uint32_t *)(rec + 1024u + (wr[0] & 63u) * 4u);
    } else if constexpr (WE == W_Q8) {
      const uint8_t *rec = p.W + ((size_t)(wr[0] >> 6) * p.wG + (kc >> 6)) * 4224u;
      const uint8_t *src = rec + (wr[0] & 63u) * 64u + ((kc >> 5) & 1u) * 32u + bw0 * 4u;
#pragma unroll
      for (int h = 0; h < UW / 4; h++) {
        u32x4 v = *(const u32x4 *)(src + 16 * h);
        br.code[4 * h] = v.x; br.code[4 * h + 1] = v.y; br.code[4 * h + 2] = v.z; br.code[4 * h + 3] = v.w;
      }
      br.s = *(const uint32_t *)(rec + 4096u + (wr[0] & 62u) * 2u);
    } else {
#pragma unroll
      for (int c = 0; c < T::BCH; c++) {
        const uint8_t *src = p.W + ((size_t)wr[c] * p.wG + kc + 8 * akc) * 2;
        if constexpr (AL) {
          br.v[c] = *(const u32x4 *)src;
        } else {
          u32x2 lo = *(const u32x2 *)src, hi = *(const u32x2 *)(src + 8);
          br.v[c] = (u32x4){lo.x, lo.y, hi.x, hi.y};
        }
      }
    }
  };
  auto store = [&](const Regs &R, int stage) __attribute__((always_inline)) {
    const u32x4 *ar = R.ar;
    const BRegs<WE, TBN> &br = R.br;
    f16 *sA = s0 + stage * T::STAGE, *sB = sA + TBM * BK;
#pragma unroll
    for (int c = 0; c < T::ACH; c++) *(u32x4 *)(sA + lds_off((tid >> 2) + (NT / 4) * c, akc)) = xperm<WE>(ar[c]);
    if constexpr (WE == W_Q4) {
      const bool fast = q4_fast_ok(br.sm);
#pragma unroll
      for (int u = 0; u < UW; u++) {
        f16x2 o[4];
        dq_q4_word(br.code[u], br.sm, fast, o);
        *(u32x4 *)(sB + lds_off(brow, bw0 + u)) = (u32x4){as_u(o[0]), as_u(o[1]), as_u(o[2]), as_u(o[3])};
      }
    } else if constexpr (WE == W_Q8) {
      const uint32_t sh = (wr[0] & 1u) ? (br.s >> 16) : (br.s & 0xffffu);
      const f16x2 s2 = as_h2(sh | (sh << 16));
#pragma unroll
      for (int u = 0; u < UW; u += 2) {
        f16x2 o[4];
        dq_q8_word(br.code[u], s2, o + 0);
        dq_q8_word(br.code[u + 1], s2, o + 2);
        *(u32x4 *)(sB + lds_off(brow, (bw0 + u) >> 1)) = (u32x4){as_u(o[0]), as_u(o[1]), as_u(o[2]), as_u(o[3])};
      }
    } else {
#pragma unroll
      for (int c = 0; c < T::BCH; c++) *(u32x4 *)(sB + lds_off((tid >> 2) + (NT / 4) * c, akc)) = br.v[c];
    }
  };

  f32x16 acc[T::BI][T::BJ];
#pragma unroll
  for (int i = 0; i < T::BI; i++)
#pragma unroll
    for (int j = 0; j < T::BJ; j++) acc[i][j] = (f32x16){};

  // MFMA operand reads: lane l reads row l%32 (+32 i) of the wave's block, chunk 2*sub + l/32; rows of one lane differ
  // by multiples of 32, so the swizzle (bits 2-3 of the row) is a per-lane constant
  const int wm = wave >> 1, wn = wave & 1, l32 = lane & 31, swz = (l32 >> 2) & 3;
  const int rdA = (wm * T::WTM + l32) * BK, rdB = TBM * BK + (wn * T::WTN + l32) * BK;
  const uint32_t nk = p.K / BK;
  // one step of MFMAs on LDS stage `cur`: both 16-k sub-steps' operands are read first, so the second sub-step's
  // reads overlap the first sub-step's MFMAs
  auto mfma_step = [&](int cur) __attribute__((always_inline)) {
    const f16 *st = s0 + cur * T::STAGE;
    if constexpr (T::FRAG2) {
      f16x8 a[2][T::BI], b[2][T::BJ];
#pragma unroll
      for (int sub = 0; sub < 2; sub++) {
        const int co = (((2 * sub + (lane >> 5)) ^ swz) & 3) * 8;
#pragma unroll
        for (int i = 0; i < T::BI; i++) a[sub][i] = *(const f16x8 *)(st + rdA + i * 32 * BK + co);
#pragma unroll
        for (int j = 0; j < T::BJ; j++) b[sub][j] = *(const f16x8 *)(st + rdB + j * 32 * BK + co);
      }
#pragma unroll
      for (int sub = 0; sub < 2; sub++)
#pragma unroll
        for (int i = 0; i < T::BI; i++)
#pragma unroll
          for (int j = 0; j < T::BJ; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[sub][i], b[sub][j], acc[i][j], 0, 0, 0);
    } else {
#pragma unroll
      for (int sub = 0; sub < 2; sub++) {
        const int co = (((2 * sub + (lane >> 5)) ^ swz) & 3) * 8;
        f16x8 a[T::BI], b[T::BJ];
#pragma unroll
        for (int i = 0; i < T::BI; i++) a[i] = *(const f16x8 *)(st + rdA + i * 32 * BK + co);
#pragma unroll
        for (int j = 0; j < T::BJ; j++) b[j] = *(const f16x8 *)(st + rdB + j * 32 * BK + co);
#pragma unroll
        for (int i = 0; i < T::BI; i++)
#pragma unroll
          for (int j = 0; j < T::BJ; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
      }
    }
  };
  // Loads and LDS writes are unconditional (past the last step they reload the last step and write the idle stage),
  // so the compiler can count outstanding loads exactly and wait only for the step it writes.
  const uint32_t klast = nk ? (nk - 1) * BK : 0;
  auto kclamp = [&](uint32_t k) { return k < klast ? k : klast; };
  if constexpr (T::PF2) {
    // loads run two steps ahead of the MFMAs: registers R0 / R1 alternate, LDS stages alternate
    Regs R0, R1;
    auto step = [&](uint32_t kt, Regs &Rnext2, const Regs &Rnext) __attribute__((always_inline)) {
      load(Rnext2, kclamp((kt + 2) * BK));
      __builtin_amdgcn_sched_barrier(0);   // keep the loads at the top of the step (issued before the MFMAs)
      mfma_step(kt & 1);
      __builtin_amdgcn_sched_barrier(0);
      store(Rnext, (kt & 1) ^ 1);
      __syncthreads();
    };
    if (nk) {
      load(R0, 0);
      load(R1, kclamp(BK));
      store(R0, 0);
    }
    __syncthreads();
    for (uint32_t kt = 0; kt < nk; kt += 2) {
      step(kt, R0, R1);
      if (kt + 1 < nk) step(kt + 1, R1, R0);
    }
  } else {
    // one step ahead (the 256 x 256 tile has no registers for a second set)
    Regs R;
    if (nk) {
      load(R, 0);
      store(R, 0);
    }
    __syncthreads();
    for (uint32_t kt = 0; kt < nk; kt++) {
      load(R, kclamp((kt + 1) * BK));
      __builtin_amdgcn_sched_barrier(0);
      mfma_step(kt & 1);
      __builtin_amdgcn_sched_barrier(0);
      store(R, (kt & 1) ^ 1);
      __syncthreads();
    }
  }

  // ---- accumulators -> LDS one 128 x 128 quadrant at a time (32x32 block layout: lane l, register r -> row
  //      8*(r/4) + 4*(l/32) + r%4, column l%32), then the epilogue over that quadrant
#pragma unroll
  for (int v = 0; v < TBM / 128; v++)
#pragma unroll
    for (int h = 0; h < TBN / 128; h++) {
      const int r0 = wm * T::WTM - v * 128, c0 = wn * T::WTN - h * 128;
      if (r0 >= 0 && r0 < 128 && c0 >= 0 && c0 < 128) {
#pragma unroll
        for (int i = 0; i < T::BI; i++)
#pragma unroll
          for (int j = 0; j < T::BJ; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
              int row = r0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
              sC[row * LDC + c0 + j * 32 + l32] = acc[i][j][r];
            }
      }
      __syncthreads();
      epilogue<NT>(p, sC, LDC, 128, mB + v * 128, nB + h * 128, tid);
      if (v + 1 < TBM / 128 || h + 1 < TBN / 128) __syncthreads();
    }
}

template <int WE, int XM, int TBM, int TBN, bool AL>
static hipError_t launch_one(const Params &p, hipStream_t s) {
  Params q = p;
  q.tilesM = (p.M + TBM - 1) / TBM;
  q.tilesN = (p.N + TBN - 1) / TBN;
  dim3 grid(q.tilesM * q.tilesN);
  hipLaunchKernelGGL((k_gemm_mfma<WE, XM, TBM, TBN, AL>), grid, dim3(NT), 0, s, q);
  return hipGetLastError();
}

template <int WE, int XM, bool AL>
static hipError_t launch_tile_al(const Params &p, unsigned bm, unsigned bn, hipStream_t s) {
  if (bm == 256 && bn == 256) return launch_one<WE, XM, 256, 256, AL>(p, s);
  if (bm == 256 && bn == 128) return launch_one<WE, XM, 256, 128, AL>(p, s);
  if (bm == 128 && bn == 256) return launch_one<WE, XM, 128, 256, AL>(p, s);
  if (bm == 128 && bn == 128) return launch_one<WE, XM, 128, 128, AL>(p, s);
  return hipErrorInvalidValue;
}

template <int WE, int XM>
static hipError_t launch_tile(const Params &p, unsigned bm, unsigned bn, hipStream_t s) {
  if constexpr (WE == W_F16 || XM == X_F16) {
    const bool al = (XM != X_F16 || (p.flags & F_XALIGN8)) && (WE != W_F16 || (p.flags & F_WALIGN8));
    if (!al) return launch_tile_al<WE, XM, false>(p, bm, bn, s);
  }
  return launch_tile_al<WE, XM, true>(p, bm, bn, s);
}

template <int WE>
static hipError_t launch_x(const Params &p, int xm, unsigned bm, unsigned bn, hipStream_t s) {
  switch (xm) {
  case X_F16: return launch_tile<WE, X_F16>(p, bm, bn, s);
  case X_LNMOD: return launch_tile<WE, X_LNMOD>(p, bm, bn, s);
  case X_RMS: return launch_tile<WE, X_RMS>(p, bm, bn, s);
  case X_CONV: return launch_tile<WE, X_CONV>(p, bm, bn, s);
  case X_CONV3: return launch_tile<WE, X_CONV3>(p, bm, bn, s);
  }
  return hipErrorInvalidValue;
}

// The tile: the largest that still gives the CUs work. Larger tiles do less dequant / prologue work and read less
// LDS per MFMA (128 x 256 with two workgroups per CU measures best; 256 x 256 runs one wave per SIMD and hides less
// latency); when the grid would leave CUs idle (or a large part of the last round of workgroups empty), smaller
// tiles win. Each candidate is scored by its relative per-CU rate times the fraction of workgroup slots (one per CU
// for 256 x 256, two for the others) that hold real work over the rounds the grid needs.
void mfma_tile(uint32_t M, uint32_t N, unsigned cus, unsigned *bm, unsigned *bn) {
  // relative rates measured on MI355X (4096^3, f16 / q4 / q8 weights, f16 / rms / lnmod prologues)
  struct C { unsigned m, n, per_cu; double rate; } cand[] = {
      {128, 256, 2, 1.0}, {256, 128, 2, 0.92}, {256, 256, 1, 0.9}, {128, 128, 2, 0.75}};
  double best = -1.0;
  for (const C &c : cand) {
    if (c.n == 256 && N <= 128) continue;
    if (c.m == 256 && M <= 128) continue;
    const uint64_t tiles = (uint64_t)((M + c.m - 1) / c.m) * ((N + c.n - 1) / c.n), slots = (uint64_t)cus * c.per_cu;
    const double rounds = (double)((tiles + slots - 1) / slots);
    const double useful = (double)M * N / ((double)c.m * c.n * rounds * slots);
    const double score = c.rate * useful;
    if (score > best + 1e-9) { best = score; *bm = c.m; *bn = c.n; }
  }
}

hipError_t launch_gemm_mfma(const Params &p, int we, int xm, unsigned bm, unsigned bn, hipStream_t s) {
  switch (we) {
  case W_Q4: return launch_x<W_Q4>(p, xm, bm, bn, s);
  case W_Q8: return launch_x<W_Q8>(p, xm, bm, bn, s);
  case W_F16: return launch_x<W_F16>(p, xm, bm, bn, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace p0k
