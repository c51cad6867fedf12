// p0k_gemv.hip — the decode path of `gemm` (M <= 16): memory-bound, so it is shaped around HBM, not the matrix cores.
//
// Work items are (N-tile of 128 ws columns) x (K-slice). 128 ws columns are two 64-row record blocks of FORMAT.md
// (for SwiGLU: 64 gate rows + the 64 matching up rows). Large N runs one slice per tile (S = 1); the host raises S
// only when there are too few tiles to occupy the GPU or X' of the slice would not fit in LDS.
//
// An item is 8 waves = 2 column halves x 4 K-quarters. Lane l of a wave owns ONE weight row: per 32-k (q4, f16) or
// 64-k (q8) unit it reads that row's codes with one 128-bit load (a wave reads a whole 1 KB / 4 KB record row-block,
// coalesced) plus the row's scale word. Each wave streams its K range through a ring of PF units held in registers:
// as soon as unit j is reduced its slot is refilled with unit j + PF, so PF loads stay in flight for the whole stream.
// Every lane owns its own sum, so the stream has no cross-lane work and no barrier; the K-quarters meet in LDS at the
// end. X' (the prologue applied, rounded to fp16 as in the reference) is staged in LDS once per item.
//
// The reduction never materialises fp16 weights; the decode is the VALU cost of this kernel, so it is kept to five
// bit operations per 8 codes. For a q4 unit with codes q, scale s, minimum mn and the unit's X':
//     sum_k x_k (q_k s + mn) = s * sum_k x_k q_k + mn * X,          X = sum_k x_k
//     sum_k x_k q_k = (Dlo - 1024 Xlo) + (Dhi - 1024 Xhi) / 16
// where the nibbles in bits 0-3 of a byte give the fp16 1024 + q (code | 0x6400), those in bits 4-7 give 1024 + 16 q
// in place (no shift), Dlo / Dhi are v_dot2_f32_f16 sums over those pairs, and Xlo / Xhi are X' sums over the same
// positions, computed once per item. q8: sum_k x_k q_k s = s * (D - 1152 X) with (byte ^ 0x80) | 0x6400 = 1152 + q.
// This is the reference's CPU path (cpuGemm over fp32 dequantised weights, test/kernels.test.js:29) in fp32; the
// reference kernel rounds each weight to fp16 first, and the two differ by less than that rounding. For x a unit
// vector it returns f16(f32(q*s + mn)) / f16(q*s) exactly, the reference's dequantised weight.
//
// With S > 1 the slices of a tile meet through a workspace: each item writes its fp32 partial tile to the memory side,
// bumps the tile's counter, and the item that arrives last sums the S partials in slice order 0..S-1 (the result does
// not depend on which item finishes last), runs the epilogue and resets the counter to 0.
#include "p0k_device.h"
#include "p0k_launch.h"

#include <type_traits>

namespace p0k {

#ifndef P0K_GV_KSUB
#define P0K_GV_KSUB 4
#endif
constexpr int GV_KSUB = P0K_GV_KSUB, GV_NT = 2 * GV_KSUB * 64;     // 512 threads
#ifndef P0K_GV_LDS_KB
#define P0K_GV_LDS_KB 40
#endif
constexpr int GV_LDS = P0K_GV_LDS_KB * 1024;
                       // X' of the slice and its group sums, then the partials

template <int WE>
struct Unit;
template <>
struct Unit<W_Q4> { static constexpr int UK = 32, PF = 4; u32x4 code; uint32_t sm; };
template <>
struct Unit<W_Q8> { static constexpr int UK = 64, PF = 4; u32x4 code[4]; uint32_t s; };
template <>
struct Unit<W_F16> { static constexpr int UK = 32, PF = 4; u32x4 v[4]; };

// longest slice whose X' (2 B per k and row) and group sums (2 floats per 32 k and row) fit the LDS budget
template <int MT>
constexpr int ks_max() { return (GV_LDS * 8 / (MT * 18)) & ~1023; }

// q4 with 4, 8 or 16 rows (MX): the unit's dot products run on the matrix cores as v_mfma_f32_4x4x4_16b_f16 with the
// lane's own weight row as the B column (below); X' rows padded by 16 bytes, and a larger LDS budget so that K = 4096
// (8192 at 4 rows) needs no split
#ifndef P0K_MX_PF
#define P0K_MX_PF 4
#endif
#ifndef P0K_MX_PX
#define P0K_MX_PX 4
#endif
template <int WE, int MT>
constexpr bool gv_mx() { return WE == W_Q4 && MT >= 4; }
template <int MT>
constexpr int mx_ksm() { return MT == 4 ? 8192 : 4096; }
template <int MT>
constexpr int mx_lds() { return MT * (mx_ksm<MT>() + 8) * 2 + mx_ksm<MT>() / 32 * MT * 4; }

// The ws column (0..127 inside a tile) that half `h` (a 64-row record block) and row j of it stand for. With the SwiGLU
// interleave the ws columns alternate gate and up rows, so half 0 takes the even columns (64 consecutive gate rows) and
// half 1 the odd ones (the matching up rows): every 128-bit load of a wave then covers one whole 1 KB record row-block,
// as without the interleave, instead of halves of two records far apart (same box: M = 1 13.53 -> 13.44 us, M = 2
// 14.5 -> 14.25, M = 4 15.09 -> 14.98; k_gemv_mq4 at 8 and 16 rows unchanged).
// The partials go to LDS in ws column order, so the finish is the same either way.
__device__ __forceinline__ uint32_t tile_col(const Params &p, uint32_t h, uint32_t j) {
  return p.epi == E_SWIGLU ? 2u * j + h : 64u * h + j;
}

// One call's tile without a K split, for the element-wise epilogues (f16, f32, bias, resadd, swiglu): one thread per
// output element sums the element's K-quarters (in quarter order, as finish() does) and applies the epilogue, so the
// tile needs no summing pass of its own and every thread has a few instructions of work (the 16-byte-store epilogue
// of finish() gives 8 threads 8 outputs each per row, a long serial tail at the end of the stream).
template <int MT, int KQ = GV_KSUB, int NT = GV_NT, int TW = 128>
__device__ __forceinline__ void finish_fast(const Params &p, const float *sR, uint32_t nB, int tid) {
  constexpr uint32_t HW = TW / 2;
  const uint32_t rows = p.M < (uint32_t)MT ? p.M : (uint32_t)MT;
  auto qsum = [&](uint32_t m, uint32_t c) {
    float s = sR[m * 128 + c];
#pragma unroll
    for (int q = 1; q < KQ; q++) s += sR[(q * MT + m) * 128 + c];
    return s;
  };
  if (p.epi == E_SWIGLU) {                                                        // gemm.js:204-210
    const uint32_t Nout = p.N >> 1;
    const bool bias = p.flags & F_BIAS, gelu = p.flags & F_GELU;
    for (uint32_t t = tid; t < rows * HW; t += NT) {
      const uint32_t m = t / HW, c = t % HW, o = (nB >> 1) + c;
      if (o >= Nout) continue;
      float gt = qsum(m, 2 * c), u = qsum(m, 2 * c + 1);
      if (bias) { gt += p.BV[p.bvOff + o]; u += p.BV[p.bvOff + p.bvUp + o]; }
      ((uint16_t *)p.Y)[(size_t)m * p.ldy + p.ny0 + o] = h_bits(glu_act(gt, gelu) * u);
    }
    return;
  }
  for (uint32_t t = tid; t < rows * TW; t += NT) {
    const uint32_t m = t / TW, c = t % TW, col = nB + c;
    if (col >= p.N) continue;
    const float v = qsum(m, c);
    const size_t yi = (size_t)m * p.ldy + p.ny0 + col;
    if (p.epi == E_F16) {                                                         // gemm.js:194-196
      ((uint16_t *)p.Y)[yi] = h_bits(v);
    } else if (p.epi == E_F32) {
      ((float *)p.Y)[yi] = v;
    } else if (p.epi == E_BIAS) {                                                 // gemm.js:211-215
      float r = v + p.EV[p.evOff + col];
      if (p.flags & F_RES) r += h_val(((const uint16_t *)p.Y)[yi]);
      ((uint16_t *)p.Y)[yi] = h_bits(r);
    } else {                                                                      // resadd, gemm.js:197-203
      const float g = (p.flags & F_GATE) ? p.EV[p.evOff + col] : 1.0f;
      const float b = (p.flags & F_BIAS) ? p.BV[p.bvOff + col] : 0.0f;
      float *y = (float *)p.Y + yi;
      *y = ((p.flags & F_STORE) ? 0.0f : *y) + g * (v + b);
    }
  }
}

__device__ __forceinline__ bool fast_epi(const Params &p, uint32_t S) {
  return S == 1 && p.epi != E_HEADS && p.epi != E_ONORMGATE;
}

// After the stream: the K-quarter partials of the item are in sR as [quarter][m][128 ws columns]; sum them, meet the
// other slices of the tile when S > 1, and run the epilogue.
template <int MT, int KQ = GV_KSUB, int NT = GV_NT>
__device__ __forceinline__ void finish(const Params &p, float *sR, float *part, uint32_t *cnt, uint32_t S, uint32_t tile,
                                       uint32_t slice, uint32_t nB, int tid, uint32_t *sLast_) {
  uint32_t &sLast = *sLast_;
  for (int t = tid; t < MT * 128; t += NT) {
    float s = sR[t];
#pragma unroll
    for (int q = 1; q < KQ; q++) s += sR[q * MT * 128 + t];
    sR[t] = s;
  }
  __syncthreads();

  if (S > 1) {
    // partial tile -> workspace [slice][m][ws column, padded to whole tiles]. The partials, the counter and the reads
    // of the last item all go to the memory side (system-coherent accesses that skip the per-XCD L2s), so items on
    // different XCDs meet without any L2 writeback or invalidation: a store is acknowledged only once it is there,
    // and every thread waits for its acknowledgements before the barrier that precedes the counter update. Partials
    // move in 16-byte vectors; workspace offsets are 32-bit (the host keeps the workspace below 4 GiB). What a split
    // costs is the chain at the end of the last item of a tile (store, acknowledgement, counter, loads: each a trip to
    // memory), about 3 us per call whatever the partials' size, so the host splits only to fill the GPU.
    const uint32_t Np = gridDim.x / S * 128u;
    const uint32_t rows = p.M < (uint32_t)MT ? p.M : (uint32_t)MT;
    const srsrc pr = stream_rsrc((const uint8_t *)part);
    for (uint32_t t = tid; t < rows * 32; t += NT) {
      const uint32_t m = t >> 5, c = (t & 31) * 4;
      sys_store128(pr, ((slice * p.M + m) * Np + nB + c) * 4u, *(const u32x4 *)(sR + m * 128 + c));
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
      uint32_t old = __hip_atomic_fetch_add(cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      sLast = (old == S - 1u) ? 1u : 0u;
    }
    __syncthreads();
    if (!sLast) return;
    for (uint32_t t = tid; t < rows * 32; t += NT) {
      const uint32_t m = t >> 5, c = (t & 31) * 4;
      f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
      for (uint32_t q = 0; q < S; q++) s += __builtin_bit_cast(f32x4, sys_load128(pr, ((q * p.M + m) * Np + nB + c) * 4u));
      *(f32x4 *)(sR + m * 128 + c) = s;
    }
    if (tid == 0) __hip_atomic_store(cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __syncthreads();
  }
  epilogue<NT>(p, sR, 128, MT, 0u, nB, tid);
}

// NARROW: items of 64 ws columns (one record block) with the 8 waves as 8 K-eighths, for calls whose 128-column
// tiles would fill only half the GPU: twice the items without a K split (S = 1 and the element-wise epilogues only).
template <int WE, int XM, int MT, bool NARROW = false>
__global__ __launch_bounds__(GV_NT) void k_gemv(Params p, float *part, uint32_t *cnt, uint32_t S, uint32_t KS) {
  static_assert(!NARROW || (WE == W_Q4 && MT <= 4), "narrow items: q4 with up to 4 rows");
  constexpr int KQ = NARROW ? 2 * GV_KSUB : GV_KSUB, TW = NARROW ? 64 : 128;   // K parts per item, item width
  constexpr bool MX = gv_mx<WE, MT>();
  constexpr int UK = Unit<WE>::UK, PF = MX ? P0K_MX_PF : Unit<WE>::PF, KSM = MX ? mx_ksm<MT>() : ks_max<MT>(), NGM = KSM / UK;
  constexpr int XSTR = MX ? KSM + 8 : KSM;                     // halves per staged X' row
  constexpr int LDSB = MX ? mx_lds<MT>() : GV_LDS;
  static_assert(KQ * MT * 128 * 4 <= LDSB, "partials must fit the staging buffer");
  // one or two rows: the partials get their own 2-8 KB, so the waves write them as they finish their streams without
  // waiting for each other; more rows: the partials reuse the X' buffer after a barrier
  constexpr bool SEP = MT <= 2;
  __shared__ __attribute__((aligned(16))) uint8_t smem[LDSB + (SEP ? KQ * MT * 128 * 4 : 0)];
  __shared__ uint32_t sLast;
  f16 *sX = (f16 *)smem;                                       // [MT][XSTR] X', pair order of the encoding
  f32x2 *sG = (f32x2 *)(smem + MT * XSTR * 2);                 // [MT][KSM / UK] (Xlo, Xhi) per unit
  float *sGx = (float *)(smem + MT * XSTR * 2);                // MX: [KSM / UK][MT] X = Xlo + Xhi per unit and row
  float *sR = (float *)(smem + (SEP ? GV_LDS : 0));            // after the stream: partials

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ch = NARROW ? 0 : wave / GV_KSUB, sub = NARROW ? wave : wave % GV_KSUB;
  const uint32_t tile = blockIdx.x / S, slice = blockIdx.x - tile * S;
  const uint32_t nB = tile * (uint32_t)TW, kb0 = slice * KS;
  const uint32_t wsc = NARROW ? (uint32_t)lane : tile_col(p, (uint32_t)ch, (uint32_t)lane);
  const uint32_t r = wrow(p, nB + wsc);
  const uint32_t nuw = KS / UK / KQ;                           // units of this wave
  const uint32_t u0 = sub * nuw;                               // its first unit inside the slice

  // byte offset of this lane's first unit from the tensor start: 32-bit (the host routes tensors of 4 GiB or more to
  // the MFMA kernel), so every load is the uniform base plus one per-lane offset, advanced by a constant per unit
  uint32_t woff;
  if constexpr (WE == W_Q4) woff = ((r >> 6) * p.wG + ((p.wk0 + kb0) >> 5)) * 1280u + (r & 63u) * 16u;
  else if constexpr (WE == W_Q8) woff = ((r >> 6) * p.wG + ((p.wk0 + kb0) >> 6)) * 4224u + (r & 63u) * 64u;
  else woff = (r * p.wG + p.wk0 + kb0) * 2u;
  constexpr uint32_t USTRIDE = WE == W_Q4 ? 1280u : WE == W_Q8 ? 4224u : 64u;

  const uint32_t sadj = 1024u - (r & 63u) * 12u;             // q4: code row -> scale word of row r in the record
  const srsrc wr = stream_rsrc(p.W);
  auto load = [&](Unit<WE> &u, uint32_t unit) {
    const uint32_t o = woff + unit * USTRIDE;                  // 32-bit offsets from the uniform base
    if constexpr (WE == W_Q4) {
      u.code = sload128(wr, o);
      u.sm = sload32(wr, o + sadj);                            // scale word r
    } else if constexpr (WE == W_Q8) {
#pragma unroll
      for (int i = 0; i < 4; i++) u.code[i] = sload128(wr, o + 16u * i);
      u.s = sload32(wr, o + 4096u - (r & 63u) * 64u + (r & 62u) * 2u);
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) u.v[i] = sload128(wr, o + 16u * i);
    }
  };

  // the nibble masks and the fp16 exponent in registers, so each pair is one v_and_or_b32 (gfx9 VOP3 takes no
  // literal operands)
  uint32_t mlo = 0x000F000Fu, mhi = 0x00F000F0u, mag = 0x64006400u;
  asm volatile("" : "+v"(mlo), "+v"(mhi), "+v"(mag));

  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; m++) acc[m] = 0.0f;

  auto compute = [&](const Unit<WE> &u, uint32_t unit) {
    const f16 *xs = sX + unit * UK;
    if constexpr (MX) {
      // 16 blocks of 4 x 4 x 4: lane l supplies B column (weight row of the lane) of block l / 4 and A row l % 4 (X'
      // row 4 g + l % 4, the same 4 rows for every block), and receives D[m = 4 g + r][its weight row], r = 0..3. B
      // holds q and 16 q (the magic-biased halves minus 1024, exact), X' at the high-nibble positions is staged as
      // x / 16, so one chain over the unit's 8 steps of 4 k returns sum x q; then y += s (sum x q) + mn X in fp32, as
      // in the dot-product form below. (Started from -G1 on the biased codes instead, the chain's partial sums sit
      // near 1024 X and its eight fp32 roundings there cost more than the fp32 sums of the other decode kernels.)
      const uint32_t wd[4] = {u.code.x, u.code.y, u.code.z, u.code.w};
      const f16x2 k1024 = {(f16)1024.0f, (f16)1024.0f};
      uint32_t h[16];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t w8 = wd[i] >> 8;
        h[4 * i + 0] = as_u(as_h2((wd[i] & mlo) | mag) - k1024);
        h[4 * i + 1] = as_u(as_h2((wd[i] & mhi) | mag) - k1024);
        h[4 * i + 2] = as_u(as_h2((w8 & mlo) | mag) - k1024);
        h[4 * i + 3] = as_u(as_h2((w8 & mhi) | mag) - k1024);
      }
      const f16x2 sm2 = as_h2(u.sm);
      const float s = (float)sm2.x, mn = (float)sm2.y;
#pragma unroll
      for (int g = 0; g < MT / 4; g++) {
        const u32x4 *x4 = (const u32x4 *)(xs + (4 * g + (lane & 3)) * XSTR);
        const f32x4 g2 = *(const f32x4 *)(sGx + unit * MT + 4 * g);
        f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const u32x4 xv = x4[i];
          d = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(f16x4, (u32x2){xv.x, xv.y}),
                                                 __builtin_bit_cast(f16x4, (u32x2){h[4 * i + 0], h[4 * i + 1]}), d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(f16x4, (u32x2){xv.z, xv.w}),
                                                 __builtin_bit_cast(f16x4, (u32x2){h[4 * i + 2], h[4 * i + 3]}), d, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) acc[4 * g + r] = fmaf(s, d[r], fmaf(mn, g2[r], acc[4 * g + r]));
      }
    } else if constexpr (WE == W_Q4) {
      const uint32_t wd[4] = {u.code.x, u.code.y, u.code.z, u.code.w};
      uint32_t h[16];                                           // per word: (q0,q4) (16q1,16q5) (q2,q6) (16q3,16q7)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t w8 = wd[i] >> 8;
        h[4 * i + 0] = (wd[i] & mlo) | mag;
        h[4 * i + 1] = (wd[i] & mhi) | mag;
        h[4 * i + 2] = (w8 & mlo) | mag;
        h[4 * i + 3] = (w8 & mhi) | mag;
      }
      const f16x2 sm2 = as_h2(u.sm);
      const float s = (float)sm2.x, mn = (float)sm2.y;
#pragma unroll
      for (int m = 0; m < MT; m++) {
        const u32x4 *x4 = (const u32x4 *)(xs + m * KSM);
        float dlo = 0.0f, dhi = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const u32x4 xv = x4[i];
          dlo = __builtin_amdgcn_fdot2(as_h2(h[4 * i + 0]), as_h2(xv.x), dlo, false);
          dhi = __builtin_amdgcn_fdot2(as_h2(h[4 * i + 1]), as_h2(xv.y), dhi, false);
          dlo = __builtin_amdgcn_fdot2(as_h2(h[4 * i + 2]), as_h2(xv.z), dlo, false);
          dhi = __builtin_amdgcn_fdot2(as_h2(h[4 * i + 3]), as_h2(xv.w), dhi, false);
        }
        const f32x2 g = sG[m * NGM + unit];
        const float t = fmaf(-1024.0f, g.x, dlo) + 0.0625f * fmaf(-1024.0f, g.y, dhi);   // sum x q, exact for e_k
        acc[m] = fmaf(s, t, fmaf(mn, g.x + g.y, acc[m]));
      }
    } else if constexpr (WE == W_Q8) {
      uint32_t h[32];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t wd[4] = {u.code[i].x ^ 0x80808080u, u.code[i].y ^ 0x80808080u, u.code[i].z ^ 0x80808080u,
                                u.code[i].w ^ 0x80808080u};
#pragma unroll
        for (int j = 0; j < 4; j++) {
          h[8 * i + 2 * j + 0] = perm(0x64646464u, wd[j], 0x04020400u);   // (1152 + q0, 1152 + q2)
          h[8 * i + 2 * j + 1] = perm(0x64646464u, wd[j], 0x04030401u);   // (1152 + q1, 1152 + q3)
        }
      }
      const uint32_t sh = (r & 1u) ? (u.s >> 16) : (u.s & 0xffffu);
      const float s = (float)__builtin_bit_cast(f16, (uint16_t)sh);
#pragma unroll
      for (int m = 0; m < MT; m++) {
        const u32x4 *x4 = (const u32x4 *)(xs + m * KSM);
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const u32x4 xv = x4[i];
          d = __builtin_amdgcn_fdot2(as_h2(h[4 * i + 0]), as_h2(xv.x), d, false);
          d = __builtin_amdgcn_fdot2(as_h2(h[4 * i + 1]), as_h2(xv.y), d, false);
          d = __builtin_amdgcn_fdot2(as_h2(h[4 * i + 2]), as_h2(xv.z), d, false);
          d = __builtin_amdgcn_fdot2(as_h2(h[4 * i + 3]), as_h2(xv.w), d, false);
        }
        const f32x2 g = sG[m * NGM + unit];
        acc[m] = fmaf(s, fmaf(-1152.0f, g.x + g.y, d), acc[m]);
      }
    } else {
#pragma unroll
      for (int m = 0; m < MT; m++) {
        const u32x4 *x4 = (const u32x4 *)(xs + m * KSM);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const u32x4 xv = x4[i];
          acc[m] = __builtin_amdgcn_fdot2(as_h2(u.v[i].x), as_h2(xv.x), acc[m], false);
          acc[m] = __builtin_amdgcn_fdot2(as_h2(u.v[i].y), as_h2(xv.y), acc[m], false);
          acc[m] = __builtin_amdgcn_fdot2(as_h2(u.v[i].z), as_h2(xv.z), acc[m], false);
          acc[m] = __builtin_amdgcn_fdot2(as_h2(u.v[i].w), as_h2(xv.w), acc[m], false);
        }
      }
    }
  };

  // This thread's first chunks of X (one; four with the matrix-core form, whose 4 rows take four) are loaded before
  // the ring: loads return in issue order (one vmcnt counter per wave), so an X load issued after the ring would wait
  // for the ring's first units and hold the staging back.
  constexpr int PX = MX ? P0K_MX_PX : 1;
  const uint32_t nb = KS / 8, nx = MT * nb;
  u32x4 xv0[PX];
#pragma unroll
  for (int i = 0; i < PX; i++) {
    const uint32_t t = (uint32_t)tid + (uint32_t)(i * GV_NT), m = t / nb;
    xv0[i] = (u32x4){0u, 0u, 0u, 0u};
    if (t < nx && m < p.M) xv0[i] = xload8<XM>(p, m, RowCtx{0, 0, 0}, kb0 + 8 * (t - m * nb));
  }
  __builtin_amdgcn_sched_barrier(0);

  // fill the ring before X' is staged, so HBM works while the prologue runs (unconditionally, clamped to the wave's
  // last unit, in the refill order: the compiler then counts the loads in flight at the loop head exactly)
  Unit<WE> ring[PF];
#pragma unroll
  for (int j = 0; j < PF; j++) {
    load(ring[j], u0 + ((uint32_t)j < nuw ? (uint32_t)j : nuw - 1u));
    __builtin_amdgcn_sched_barrier(0);
  }

  // X' of the slice -> LDS in the pair order of the encoding, and per unit the X' sums over the low (even pair slot)
  // and high (odd pair slot) positions: a unit's UK / 8 chunks sit in as many adjacent lanes (nx and the thread count
  // are multiples of UK / 8, so such a lane group is active or idle as a whole), which sum across by shuffles
  auto stage = [&](uint32_t t, u32x4 v) __attribute__((always_inline)) {
    const uint32_t m = t / nb, kq = t - m * nb;
    v = xperm<WE>(v);
    if constexpr (WE != W_F16 && MX) {
      // the unit's X' sum of this row (the 4x4x4 form needs lo + hi only): v_dot2_f32_f16 against ones, 4
      // instructions instead of 8 conversions and 6 adds (M = 2: 14.0 -> 13.7 us; M = 4 14.6-14.8 -> 14.6)
      const f16x2 one2 = {(f16)1.0f, (f16)1.0f};
      float t = __builtin_amdgcn_fdot2(as_h2(v.x), one2, 0.0f, false);
      t = __builtin_amdgcn_fdot2(as_h2(v.y), one2, t, false);
      t = __builtin_amdgcn_fdot2(as_h2(v.z), one2, t, false);
      t = __builtin_amdgcn_fdot2(as_h2(v.w), one2, t, false);
      static_assert(UK / 8 == 4, "a unit's chunks are one lane quad");
      // sum over the lane quad by DPP quad permutes (xor 1, then xor 2; M = 4 14.65-14.74 -> 14.32-14.58 us)
      t += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, t), 0xB1, 0xF, 0xF, false));
      t += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, t), 0x4E, 0xF, 0xF, false));
      if (kq % (UK / 8) == 0) sGx[(kq / (UK / 8)) * MT + m] = t;
      const f16x2 r16 = {(f16)0.0625f, (f16)0.0625f};
      v.y = as_u(as_h2(v.y) * r16);
      v.w = as_u(as_h2(v.w) * r16);
    } else if constexpr (WE == W_Q4) {
      // (lo, hi) by v_dot2 against ones and DPP quad sums, as above (q4 N 4096 K 4096 at one row: 6.19 -> 6.11 us)
      const f16x2 one2 = {(f16)1.0f, (f16)1.0f};
      float lo = __builtin_amdgcn_fdot2(as_h2(v.z), one2, __builtin_amdgcn_fdot2(as_h2(v.x), one2, 0.0f, false), false);
      float hi = __builtin_amdgcn_fdot2(as_h2(v.w), one2, __builtin_amdgcn_fdot2(as_h2(v.y), one2, 0.0f, false), false);
      lo += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, lo), 0xB1, 0xF, 0xF, false));
      hi += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, hi), 0xB1, 0xF, 0xF, false));
      lo += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, lo), 0x4E, 0xF, 0xF, false));
      hi += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, hi), 0x4E, 0xF, 0xF, false));
      if (kq % (UK / 8) == 0) sG[m * NGM + kq / (UK / 8)] = (f32x2){lo, hi};
    } else if constexpr (WE != W_F16) {
      const f16x2 a = as_h2(v.x), b = as_h2(v.y), c = as_h2(v.z), d = as_h2(v.w);
      float lo = ((float)a.x + (float)a.y) + ((float)c.x + (float)c.y);
      float hi = ((float)b.x + (float)b.y) + ((float)d.x + (float)d.y);
#pragma unroll
      for (int o = 1; o < UK / 8; o *= 2) {
        lo += __shfl_xor(lo, o);
        hi += __shfl_xor(hi, o);
      }
      if constexpr (MX) {
        if (kq % (UK / 8) == 0) sGx[(kq / (UK / 8)) * MT + m] = lo + hi;
        const f16x2 r16 = {(f16)0.0625f, (f16)0.0625f};
        v.y = as_u(as_h2(v.y) * r16);
        v.w = as_u(as_h2(v.w) * r16);
      } else if (kq % (UK / 8) == 0) {
        sG[m * NGM + kq / (UK / 8)] = (f32x2){lo, hi};
      }
    }
    *(u32x4 *)(sX + m * XSTR + 8 * kq) = v;
  };
#pragma unroll
  for (int i = 0; i < PX; i++) {
    const uint32_t t = (uint32_t)tid + (uint32_t)(i * GV_NT);
    if (t < nx) stage(t, xv0[i]);
  }
  for (uint32_t t = (uint32_t)tid + (uint32_t)(PX * GV_NT); t < nx; t += GV_NT) {
    const uint32_t m = t / nb;
    stage(t, m < p.M ? xload8<XM>(p, m, RowCtx{0, 0, 0}, kb0 + 8 * (t - m * nb)) : (u32x4){0u, 0u, 0u, 0u});
  }
  __syncthreads();

  // the stream: reduce slot j, refill it with the unit PF ahead
  uint32_t j0 = 0;
#pragma unroll 1
  for (; j0 + PF <= nuw; j0 += PF) {
#pragma unroll
    for (int j = 0; j < PF; j++) {
      compute(ring[j], u0 + j0 + j);
      // refill unconditionally (past the end: the wave's last unit again, unused): a conditional refill would keep
      // the old and the new slot contents apart and double the ring's registers
      const uint32_t nx = j0 + PF + j;
      load(ring[j], u0 + (nx < nuw ? nx : nuw - 1u));
      // keep the refill here: left to itself the scheduler sinks all refills to the end of the batch behind one
      // vmcnt(0), so a batch's loads would only start after the whole batch is reduced
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int j = 0; j < PF; j++)
    if (j0 + j < nuw) compute(ring[j], u0 + j0 + j);
  if constexpr (!SEP) __syncthreads();                         // X' is dead: the buffer takes the partials

  // the K-quarters meet in LDS
#pragma unroll
  for (int m = 0; m < MT; m++) sR[(sub * MT + m) * 128 + wsc] = acc[m];
  __syncthreads();
  if constexpr (NARROW) finish_fast<MT, KQ, GV_NT, TW>(p, sR, nB, tid);     // (the host sends only S = 1 here)
  else if (fast_epi(p, S)) finish_fast<MT>(p, sR, nB, tid);
  else finish<MT>(p, sR, part, cnt, S, tile, slice, nB, tid, &sLast);
}

// ------------------------------------------------------------------------------------------------------------------
// Short decode calls (q4 or q8, 1..4 rows, element-wise epilogues): items of 16 weight rows, so that even N = 4096 gives
// one item per CU with no K split. A call of this size is mostly latency (launch, the first bytes' trip from HBM, the
// finish), and a ring per lane keeps only a few units in flight per CU; here every lane issues all of its weight loads
// at once (the whole item, 16 rows x K, is in flight on the CU right after the launch), X' is staged in LDS with its
// per-unit sums while those loads travel, and each lane reduces its units with the same algebraic form as k_gemv. The
// 8 waves take rounds of 32 consecutive units (wave w the units 4 w .. 4 w + 3 of each). q4 (32-k units of 16 bytes
// per row): lane l of a wave owns row l % 16 and unit l / 16 of every round, so one load instruction reads four
// 256-byte runs of 16 whole code rows. q8 (64-k units of 64 bytes per row): lane l owns row (l / 4) % 16 and the
// 16-byte chunk l % 4 of all four units of the round, so one load instruction reads one unit's 1 KB of code rows
// whole. The four lanes of a row meet by DPP, the waves in LDS (wave order), and one thread per output element applies
// the epilogue. With the SwiGLU interleave, rows 0..7 of an item are 8 consecutive gate rows and rows 8..15 the
// matching up rows.
constexpr int SN_NT = 512, SN_ROWS = 16;
template <int WE>
struct SnUnit;
template <>
struct SnUnit<W_Q4> { static constexpr int UK = 32, NC = 1; };
template <>
struct SnUnit<W_Q8> { static constexpr int UK = 64, NC = 4; };

// the epilogue of a short-call item: sR[wave][MT][16] holds each wave's sums of the item's 16 ws columns; the waves
// are added in wave order and one thread per output element applies the element-wise epilogue
template <int MT>
__device__ __forceinline__ void sn_epilogue(const Params &p, const float *sR, uint32_t nB, int tid) {
  const bool glu = p.epi == E_SWIGLU;
  const uint32_t rows = p.M < (uint32_t)MT ? p.M : (uint32_t)MT;
  auto tot = [&](uint32_t m, uint32_t i) {
    float v = sR[m * SN_ROWS + i];
#pragma unroll
    for (int w = 1; w < SN_NT / 64; w++) v += sR[(w * MT + m) * SN_ROWS + i];
    return v;
  };
  if (glu) {                                                                      // gemm.js:204-210
    const uint32_t Nout = p.N >> 1;
    const bool bias = p.flags & F_BIAS, gelu = p.flags & F_GELU;
    if ((uint32_t)tid < rows * 8u) {
      const uint32_t m = tid / 8, c = tid % 8, o = (nB >> 1) + c;
      if (o < Nout) {
        float gt = tot(m, c), u = tot(m, 8 + c);
        if (bias) { gt += p.BV[p.bvOff + o]; u += p.BV[p.bvOff + p.bvUp + o]; }
        ((uint16_t *)p.Y)[(size_t)m * p.ldy + p.ny0 + o] = h_bits(glu_act(gt, gelu) * u);
      }
    }
    return;
  }
  if ((uint32_t)tid < rows * SN_ROWS) {
    const uint32_t m = tid / SN_ROWS, c = tid % SN_ROWS, col = nB + c;
    if (col >= p.N) return;
    const float v = tot(m, c);
    const size_t yi = (size_t)m * p.ldy + p.ny0 + col;
    if (p.epi == E_F16) {                                                         // gemm.js:194-196
      ((uint16_t *)p.Y)[yi] = h_bits(v);
    } else if (p.epi == E_F32) {
      ((float *)p.Y)[yi] = v;
    } else if (p.epi == E_BIAS) {                                                 // gemm.js:211-215
      float rr = v + p.EV[p.evOff + col];
      if (p.flags & F_RES) rr += h_val(((const uint16_t *)p.Y)[yi]);
      ((uint16_t *)p.Y)[yi] = h_bits(rr);
    } else {                                                                      // resadd, gemm.js:197-203
      const float g = (p.flags & F_GATE) ? p.EV[p.evOff + col] : 1.0f;
      const float b = (p.flags & F_BIAS) ? p.BV[p.bvOff + col] : 0.0f;
      float *y = (float *)p.Y + yi;
      *y = ((p.flags & F_STORE) ? 0.0f : *y) + g * (v + b);
    }
  }
}

template <int WE, int XM, int MT, int RND>
__global__ __launch_bounds__(SN_NT) void k_gemv_sn(Params p) {
  constexpr int UK = SnUnit<WE>::UK, NC = SnUnit<WE>::NC, CPU_ = UK / 8;   // k per unit, code loads, 8-k chunks
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ri = WE == W_Q8 ? (lane >> 2) & 15 : lane & 15, us = WE == W_Q8 ? lane & 3 : lane >> 4;
  const bool glu = p.epi == E_SWIGLU;
  // workgroups go to the 8 XCDs in turn: give each XCD a contiguous run of items, so the four items of a 64-row record
  // block (and their shared 128-byte lines of scale words) meet in one L2 instead of four
  const uint32_t nit = gridDim.x;
  const uint32_t item = (nit & 7u) ? blockIdx.x : (blockIdx.x & 7u) * (nit >> 3) + (blockIdx.x >> 3);
  const uint32_t nB = item * (uint32_t)SN_ROWS;
  const uint32_t wsc = glu ? (ri < 8 ? 2u * ri : 2u * (ri - 8) + 1u) : (uint32_t)ri;
  const uint32_t r = wrow(p, nB + wsc);
  const uint32_t nun = p.K / UK;                               // units of the call
  // byte offset of row r's first unit and of its scale word from a unit's code row (q4: scale word r at 1024 + 4 r;
  // q8: the f16 scale of row r at 4096 + 2 r, read as the 4-byte word of its row pair)
  constexpr uint32_t USTRIDE = WE == W_Q4 ? 1280u : 4224u;
  const uint32_t woff = WE == W_Q4 ? ((r >> 6) * p.wG + (p.wk0 >> 5)) * 1280u + (r & 63u) * 16u
                                   : ((r >> 6) * p.wG + (p.wk0 >> 6)) * 4224u + (r & 63u) * 64u;
  const uint32_t sadj = WE == W_Q4 ? 1024u - (r & 63u) * 12u : 4096u - (r & 63u) * 64u + (r & 62u) * 2u;
  const srsrc wr = stream_rsrc(p.W);
  // this thread's first chunk of X before the weights (loads return in issue order: issued after them, it would wait
  // for the whole item's weights before the staging below could start)
  const uint32_t nb = p.K / 8, nx = MT * nb;                   // 8-k chunks (nx is a multiple of CPU_: whole lane groups)
  u32x4 xv0 = (u32x4){0u, 0u, 0u, 0u};
  if ((uint32_t)tid < nx && (uint32_t)tid / nb < p.M) xv0 = xload8<XM>(p, tid / nb, RowCtx{0, 0, 0}, 8 * (tid % nb));
  __builtin_amdgcn_sched_barrier(0);
  // every weight load of this lane (clamped past the last unit: the clamped ones are not reduced); q4: its unit's code
  // row and scale word; q8: its chunk of each of the round's four units (unit 4 w + c in code[rd][c]) and their scales
  u32x4 code[RND][NC];
  uint32_t sm[RND][NC];
#pragma unroll
  for (int rd = 0; rd < RND; rd++) {
#pragma unroll
    for (int c = 0; c < NC; c++) {
      uint32_t u = (uint32_t)rd * 32u + (uint32_t)wave * 4u + (uint32_t)(WE == W_Q8 ? c : us);
      u = u < nun ? u : nun - 1u;
      code[rd][c] = sload128(wr, woff + u * USTRIDE + (WE == W_Q8 ? 16u * (uint32_t)us : 0u));
      sm[rd][c] = sload32(wr, woff + u * USTRIDE + sadj);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // X' -> LDS in the pair order of the encoding, and per unit and row the X' sums (q4: over the low / high nibble
  // positions; q8: the whole unit, in .x)
  extern __shared__ __attribute__((aligned(16))) uint8_t sn_smem[];
  f16 *sX = (f16 *)sn_smem;                                    // [MT][K]
  f32x2 *sG = (f32x2 *)(sn_smem + (size_t)MT * p.K * 2);      // [MT][K / UK]
  for (uint32_t t = tid; t < nx; t += SN_NT) {
    const uint32_t m = t / nb, kq = t - m * nb;
    u32x4 v = (u32x4){0u, 0u, 0u, 0u};
    if (t == (uint32_t)tid) v = xv0;
    else if (m < p.M) v = xload8<XM>(p, m, RowCtx{0, 0, 0}, 8 * kq);
    v = xperm<WE>(v);
    const f16x2 one2 = {(f16)1.0f, (f16)1.0f};
    float lo = __builtin_amdgcn_fdot2(as_h2(v.z), one2, __builtin_amdgcn_fdot2(as_h2(v.x), one2, 0.0f, false), false);
    float hi = __builtin_amdgcn_fdot2(as_h2(v.w), one2, __builtin_amdgcn_fdot2(as_h2(v.y), one2, 0.0f, false), false);
    if constexpr (WE == W_Q8) { lo += hi; hi = 0.0f; }
    lo += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, lo), 0xB1, 0xF, 0xF, false));
    hi += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, hi), 0xB1, 0xF, 0xF, false));
    lo += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, lo), 0x4E, 0xF, 0xF, false));
    hi += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, hi), 0x4E, 0xF, 0xF, false));
    if constexpr (CPU_ == 8) lo += __shfl_xor(lo, 4);         // q8: a unit's 8 chunks are two lane quads
    if (kq % CPU_ == 0u) sG[m * (nb / CPU_) + kq / CPU_] = (f32x2){lo, hi};
    *(u32x4 *)(sX + (size_t)m * p.K + 8 * kq) = v;
  }
  __syncthreads();

  uint32_t mlo = 0x000F000Fu, mhi = 0x00F000F0u, mag = 0x64006400u;
  asm volatile("" : "+v"(mlo), "+v"(mhi), "+v"(mag));
  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; m++) acc[m] = 0.0f;
#pragma unroll
  for (int rd = 0; rd < RND; rd++) {
    if constexpr (WE == W_Q4) {
      const uint32_t u = (uint32_t)rd * 32u + (uint32_t)wave * 4u + (uint32_t)us;
      if (u >= nun) break;                                     // (units ascend with rd)
      const uint32_t wd[4] = {code[rd][0].x, code[rd][0].y, code[rd][0].z, code[rd][0].w};
      uint32_t h[16];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t w8 = wd[i] >> 8;
        h[4 * i + 0] = (wd[i] & mlo) | mag;
        h[4 * i + 1] = (wd[i] & mhi) | mag;
        h[4 * i + 2] = (w8 & mlo) | mag;
        h[4 * i + 3] = (w8 & mhi) | mag;
      }
      const f16x2 sm2 = as_h2(sm[rd][0]);
      const float s = (float)sm2.x, mn = (float)sm2.y;
#pragma unroll
      for (int m = 0; m < MT; m++) {
        const u32x4 *x4 = (const u32x4 *)(sX + (size_t)m * p.K + u * UK);
        float dlo = 0.0f, dhi = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const u32x4 xv = x4[i];
          dlo = __builtin_amdgcn_fdot2(as_h2(h[4 * i + 0]), as_h2(xv.x), dlo, false);
          dhi = __builtin_amdgcn_fdot2(as_h2(h[4 * i + 1]), as_h2(xv.y), dhi, false);
          dlo = __builtin_amdgcn_fdot2(as_h2(h[4 * i + 2]), as_h2(xv.z), dlo, false);
          dhi = __builtin_amdgcn_fdot2(as_h2(h[4 * i + 3]), as_h2(xv.w), dhi, false);
        }
        const f32x2 g = sG[m * (nb / 4u) + u];
        const float t = fmaf(-1024.0f, g.x, dlo) + 0.0625f * fmaf(-1024.0f, g.y, dhi);   // sum x q, exact for e_k
        acc[m] = fmaf(s, t, fmaf(mn, g.x + g.y, acc[m]));
      }
    } else {
      // q8: (1152 + q) in the fp16 halves (the code byte's sign bit flipped puts 128 + q in the low byte), one FMA
      // removes 1152 X, and the row's scale multiplies the unit's sum, as in k_gemv; the lane holds 16 k of the unit
      // (chunk us), and the chunk-0 lane removes the unit's 1152 X for all four
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const uint32_t u = (uint32_t)rd * 32u + (uint32_t)wave * 4u + (uint32_t)c;
        if (u >= nun) break;                                   // (units ascend with c and rd)
        uint32_t h[8];
        const uint32_t wd[4] = {code[rd][c].x ^ 0x80808080u, code[rd][c].y ^ 0x80808080u, code[rd][c].z ^ 0x80808080u,
                                code[rd][c].w ^ 0x80808080u};
#pragma unroll
        for (int j = 0; j < 4; j++) {
          h[2 * j + 0] = perm(0x64646464u, wd[j], 0x04020400u);   // (1152 + q0, 1152 + q2)
          h[2 * j + 1] = perm(0x64646464u, wd[j], 0x04030401u);   // (1152 + q1, 1152 + q3)
        }
        const uint32_t sh = (r & 1u) ? (sm[rd][c] >> 16) : (sm[rd][c] & 0xffffu);
        const float s = (float)__builtin_bit_cast(f16, (uint16_t)sh);
#pragma unroll
        for (int m = 0; m < MT; m++) {
          const u32x4 *x4 = (const u32x4 *)(sX + (size_t)m * p.K + u * UK + 16u * (uint32_t)us);
          float d = 0.0f;
#pragma unroll
          for (int i = 0; i < 2; i++) {
            const u32x4 xv = x4[i];
            d = __builtin_amdgcn_fdot2(as_h2(h[4 * i + 0]), as_h2(xv.x), d, false);
            d = __builtin_amdgcn_fdot2(as_h2(h[4 * i + 1]), as_h2(xv.y), d, false);
            d = __builtin_amdgcn_fdot2(as_h2(h[4 * i + 2]), as_h2(xv.z), d, false);
            d = __builtin_amdgcn_fdot2(as_h2(h[4 * i + 3]), as_h2(xv.w), d, false);
          }
          const float g = us == 0 ? sG[m * (nb / 8u) + u].x : 0.0f;
          acc[m] = fmaf(s, fmaf(-1152.0f, g, d), acc[m]);
        }
      }
    }
  }
  // the row's four lanes (q4: l, l + 16, l + 32, l + 48; q8: a lane quad) in a fixed order, then the waves in wave
  // order
  float *sR = (float *)sn_smem;                                // [wave][MT][16] after a barrier (X' is dead)
#pragma unroll
  for (int m = 0; m < MT; m++) {
    if constexpr (WE == W_Q8) {
      acc[m] += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, acc[m]), 0xB1, 0xF, 0xF, false));
      acc[m] += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, acc[m]), 0x4E, 0xF, 0xF, false));
    } else {
      acc[m] += __shfl_xor(acc[m], 16);
      acc[m] += __shfl_xor(acc[m], 32);
    }
  }
  __syncthreads();
  if (us == 0) {
#pragma unroll
    for (int m = 0; m < MT; m++) sR[(wave * MT + m) * SN_ROWS + ri] = acc[m];
  }
  __syncthreads();
  sn_epilogue<MT>(p, sR, nB, tid);
}

// The short-call items for f16 weights (rows of 16-byte aligned fp16, `ld` and the column offset multiples of 8): units
// of 64 k, one 128-byte run per row. Lane l of a wave owns rows (l / 8) % 8 and 8 + (l / 8) % 8 of the item and the
// 16-byte chunk l % 8 (8 k) of each unit; wave w takes the units w, w + 8, w + 16, ..., so one load instruction reads
// 8 rows x 128 bytes and every load of the item is in flight right after the launch. No X' sums: the dot products of
// fp16 pairs are the reference's fp32 weight model directly. A row's eight lanes meet by DPP and one lane shuffle.
template <int XM, int MT, int RND>
__global__ __launch_bounds__(SN_NT) void k_gemv_sn16(Params p) {
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rr = (lane >> 3) & 7, cq = lane & 7;
  const bool glu = p.epi == E_SWIGLU;
  const uint32_t nit = gridDim.x;
  const uint32_t item = (nit & 7u) ? blockIdx.x : (blockIdx.x & 7u) * (nit >> 3) + (blockIdx.x >> 3);
  const uint32_t nB = item * (uint32_t)SN_ROWS;
  uint32_t woff[2];
#pragma unroll
  for (int c = 0; c < 2; c++) {
    const uint32_t ri = (uint32_t)(rr + 8 * c);
    const uint32_t wsc = glu ? (ri < 8 ? 2u * ri : 2u * (ri - 8) + 1u) : ri;
    woff[c] = (wrow(p, nB + wsc) * p.wG + p.wk0) * 2u + 16u * (uint32_t)cq;   // 32-bit: the tensor is below 4 GiB
  }
  const srsrc wr = stream_rsrc(p.W);
  const uint32_t nun = p.K / 64;
  const uint32_t nb = p.K / 8, nx = MT * nb;
  u32x4 xv0 = (u32x4){0u, 0u, 0u, 0u};
  if ((uint32_t)tid < nx && (uint32_t)tid / nb < p.M) xv0 = xload8<XM>(p, tid / nb, RowCtx{0, 0, 0}, 8 * (tid % nb));
  __builtin_amdgcn_sched_barrier(0);
  u32x4 wv[RND][2];
#pragma unroll
  for (int rd = 0; rd < RND; rd++) {
    uint32_t u = (uint32_t)rd * 8u + (uint32_t)wave;
    u = u < nun ? u : nun - 1u;
#pragma unroll
    for (int c = 0; c < 2; c++) wv[rd][c] = sload128(wr, woff[c] + u * 128u);
  }
  __builtin_amdgcn_sched_barrier(0);

  extern __shared__ __attribute__((aligned(16))) uint8_t sn_smem[];
  f16 *sX = (f16 *)sn_smem;                                    // [MT][K]
  for (uint32_t t = tid; t < nx; t += SN_NT) {
    const uint32_t m = t / nb, kq = t - m * nb;
    u32x4 v = (u32x4){0u, 0u, 0u, 0u};
    if (t == (uint32_t)tid) v = xv0;
    else if (m < p.M) v = xload8<XM>(p, m, RowCtx{0, 0, 0}, 8 * kq);
    *(u32x4 *)(sX + (size_t)m * p.K + 8 * kq) = v;
  }
  __syncthreads();

  float acc[2][MT];
#pragma unroll
  for (int c = 0; c < 2; c++)
#pragma unroll
    for (int m = 0; m < MT; m++) acc[c][m] = 0.0f;
#pragma unroll
  for (int rd = 0; rd < RND; rd++) {
    const uint32_t u = (uint32_t)rd * 8u + (uint32_t)wave;
    if (u >= nun) break;                                       // (units ascend with rd)
#pragma unroll
    for (int m = 0; m < MT; m++) {
      const u32x4 xv = *(const u32x4 *)(sX + (size_t)m * p.K + u * 64u + 8u * (uint32_t)cq);
#pragma unroll
      for (int c = 0; c < 2; c++) {
        float d = acc[c][m];
        d = __builtin_amdgcn_fdot2(as_h2(wv[rd][c].x), as_h2(xv.x), d, false);
        d = __builtin_amdgcn_fdot2(as_h2(wv[rd][c].y), as_h2(xv.y), d, false);
        d = __builtin_amdgcn_fdot2(as_h2(wv[rd][c].z), as_h2(xv.z), d, false);
        d = __builtin_amdgcn_fdot2(as_h2(wv[rd][c].w), as_h2(xv.w), d, false);
        acc[c][m] = d;
      }
    }
  }
  // a row's eight chunk lanes (xor 1, 2 within the quad, then xor 4), then the waves in wave order
  float *sR = (float *)sn_smem;                                // [wave][MT][16] after a barrier (X' is dead)
#pragma unroll
  for (int c = 0; c < 2; c++)
#pragma unroll
    for (int m = 0; m < MT; m++) {
      float v = acc[c][m];
      v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
      v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
      v += __shfl_xor(v, 4);
      acc[c][m] = v;
    }
  __syncthreads();
  if (cq == 0) {
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
      for (int m = 0; m < MT; m++) sR[(wave * MT + m) * SN_ROWS + rr + 8 * c] = acc[c][m];
  }
  __syncthreads();
  sn_epilogue<MT>(p, sR, nB, tid);
}

// the longest K a short-call item serves (q4: rounds of 32 units up to 16 of 1024 k; q8: up to 4 rounds of 2048 k, whose
// four code loads per unit take 16 registers per round; f16: up to 16 rounds of 512 k, 8 registers each) and its LDS
// bytes
constexpr int SN_RND_Q4 = 16, SN_RND_Q8 = 4, SN_RND_F16 = 16;
unsigned gemv_sn_kmax(int we) {
  return we == W_Q8 ? SN_RND_Q8 * 32u * 64u : we == W_F16 ? SN_RND_F16 * 8u * 64u : SN_RND_Q4 * 32u * 32u;
}
// X' and its per-unit sums; after the stream the same buffer holds the waves' partials (8 waves x M x 16 floats)
uint32_t gemv_sn_lds(int we, uint32_t M, uint32_t K) {
  const uint32_t sums = we == W_F16 ? 0u : M * (K / (we == W_Q8 ? 64u : 32u)) * 8u;
  const uint32_t x = M * K * 2u + sums, r = (uint32_t)(SN_NT / 64) * M * SN_ROWS * 4u;
  return x > r ? x : r;
}

template <int XM, int MT>
static hipError_t launch_sn16_mt(const Params &p, hipStream_t s) {
  const uint32_t rounds = (p.K / 64u + 7u) / 8u;
  const uint32_t lds = gemv_sn_lds(W_F16, MT, p.K);
  const dim3 grid((p.N + SN_ROWS - 1) / SN_ROWS);
#define SN16_CASE(R) case R: hipLaunchKernelGGL((k_gemv_sn16<XM, MT, R>), grid, dim3(SN_NT), lds, s, p); break;
  switch (rounds <= 2 ? 2 : rounds <= 4 ? 4 : rounds <= 8 ? 8 : 16) {
    SN16_CASE(2) SN16_CASE(4) SN16_CASE(8) SN16_CASE(16)
  default: return hipErrorInvalidValue;
  }
#undef SN16_CASE
  return hipGetLastError();
}
template <int WE, int XM, int MT>
static hipError_t launch_sn_mt(const Params &p, hipStream_t s) {
  if constexpr (WE == W_F16) {
    return launch_sn16_mt<XM, MT>(p, s);
  } else {
    const uint32_t rounds = (p.K / (uint32_t)SnUnit<WE>::UK + 31u) / 32u;
    const uint32_t lds = gemv_sn_lds(WE, MT, p.K);
    const dim3 grid((p.N + SN_ROWS - 1) / SN_ROWS);
#define SN_CASE(R) case R: hipLaunchKernelGGL((k_gemv_sn<WE, XM, MT, R>), grid, dim3(SN_NT), lds, s, p); break;
    if constexpr (WE == W_Q4) {
      switch (rounds <= 4 ? 4 : rounds <= 8 ? 8 : rounds <= 12 ? 12 : 16) {
        SN_CASE(4) SN_CASE(8) SN_CASE(12) SN_CASE(16)
      default: return hipErrorInvalidValue;
      }
    } else {
      switch (rounds <= 2 ? 2 : 4) {
        SN_CASE(2) SN_CASE(4)
      default: return hipErrorInvalidValue;
      }
    }
#undef SN_CASE
    return hipGetLastError();
  }
}
template <int WE, int XM>
static hipError_t launch_sn_x(const Params &p, hipStream_t s) {
  if (p.M == 1) return launch_sn_mt<WE, XM, 1>(p, s);
  if (p.M == 2) return launch_sn_mt<WE, XM, 2>(p, s);
  return launch_sn_mt<WE, XM, 4>(p, s);
}
template <int WE>
static hipError_t launch_sn_w(const Params &p, int xm, hipStream_t s) {
  switch (xm) {
  case X_F16: return launch_sn_x<WE, X_F16>(p, s);
  case X_LNMOD: return launch_sn_x<WE, X_LNMOD>(p, s);
  case X_RMS: return launch_sn_x<WE, X_RMS>(p, s);
  }
  return hipErrorInvalidValue;
}
hipError_t launch_gemv_sn(const Params &p, int we, int xm, hipStream_t s) {
  const uint32_t uk = we == W_Q4 ? 32u : 64u, wk = we == W_F16 ? 8u : uk;
  if ((we != W_Q4 && we != W_Q8 && we != W_F16) || (we == W_F16 && !(p.flags & F_WALIGN8)) || p.M == 0 || p.M > 4 ||
      p.K % uk || p.K > gemv_sn_kmax(we) || p.wk0 % wk || p.epi == E_HEADS || p.epi == E_ONORMGATE ||
      gemv_sn_lds(we, p.M <= 2 ? p.M : 4, p.K) > 64u * 1024u)
    return hipErrorInvalidValue;
  return we == W_Q4 ? launch_sn_w<W_Q4>(p, xm, s) : we == W_Q8 ? launch_sn_w<W_Q8>(p, xm, s) : launch_sn_w<W_F16>(p, xm, s);
}

// ------------------------------------------------------------------------------------------------------------------
// Decode on the matrix cores (q4 with 3..16 rows when k_gemv_mq4 is switched off, M <= 16 for q8 / f16). With several rows of X the per-row dot products of the stream above
// multiply its VALU work; here the same items, waves and ring feed v_mfma_f32_16x16x32_f16 instead. Per 32-k step
// (q4, f16; 64-k for q8) a wave runs one MFMA per block of 16 of its 64 weight rows: A = X' (16 rows, zero past M),
// B = the block's weights. Lane l supplies, for block i, weight row 16 i + l%16 and the 8 k at 8 (l/16) of the step
// (one q4 code word, two q8 words or 16 f16 bytes, each load instruction covering 16 whole rows), and receives
// D[m = 4 (l/16) + r][row 16 i + l%16], r = 0..3: every lane keeps ONE weight row per block, so the row's scale and
// minimum apply in registers. The weights are never dequantised: the MFMA multiplies the magic-biased codes, as in
// the stream above, and the per-group corrections come from X' sums staged with X':
//   q4: B holds 1024 + q (low nibbles) and 1024 + 16 q (high nibbles, in place), A holds x and x / 16 at those
//       positions, so D = sum x q + G1 with G1 = 1024 X_lo + 64 X_hi; y += s (D - G1) + mn (X_lo + X_hi), the MFMA
//       starting from -G1
//   q8: B holds 1152 + q; y += s (D - 1152 X)
//   f16: B holds the weights; D accumulates across steps in the MFMA.
// This is the fp32 arithmetic of the reference's CPU path (cpuGemm over fp32 dequantised weights) like the stream
// above, and for x a unit vector it returns the dequantised weight f16(f32(q*s + mn)) / f16(q*s) exactly.
template <int WE>
struct MUnit;
template <>
struct MUnit<W_Q4> { static constexpr int UK = 32, PF = 4; u32x4 code; uint32_t sm; };   // row `lane`, as loaded
template <>
struct MUnit<W_Q8> { static constexpr int UK = 64, PF = 3; u32x4 code[4]; uint32_t s[4]; };
template <>
struct MUnit<W_F16> { static constexpr int UK = 64, PF = 3; u32x4 v[4][2]; };   // lane: 16 k (32 B) of a row

// (units in flight per wave, q8 / f16: 3; q8 with 2 / 4 / 6: 14.3 / 14.9 / 27.3 against 13.4 us at N 14336, K 4096,
// M = 1; f16 with 2 / 4: 23.8 / 34.1 against 22.7 us at N 14336, K 2048, M = 1, 11.3 / 13.6 against 11.5 at N 4096)
constexpr int MF_KSM = 4096;                                // longest K slice of one item
// X' rows are MF_KSM + 8 halfs apart: the 16 rows an MFMA A read touches then start 4 banks apart instead of all in
// one bank (8 KB rows)
constexpr int MF_KSP = MF_KSM + 8;
constexpr int MF_XG = 16 * MF_KSP * 2 + 16 * (MF_KSM / 32) * 8;    // X' of 16 rows + (G1, G2) per row and group
constexpr int MF_LDS = MF_XG + 8 * 64 * 20;                 // + per wave: one q4 unit (64 rows x 16 B) and its scales

// NARROW: items of 64 ws columns with the 8 waves as K-eighths (S = 1, element-wise epilogues), as in k_gemv
// XS (q8 / f16 with fp16 X of 16-byte rows): no X' staging; each unit's 16 X rows x 64 k (2 KB) are copied into the
// wave's LDS slot of its ring entry by two load-to-LDS instructions issued with the unit's weight loads, and q8's G1
// comes from two MFMAs against a constant B operand, as in k_gemv_mq4
template <int WE, int XM, bool NARROW = false, bool XS = false>
__global__ __launch_bounds__(GV_NT) void k_gemv_mf(Params p, float *part, uint32_t *cnt, uint32_t S, uint32_t KS) {
  constexpr int MT = 16, KQ = NARROW ? 2 * GV_KSUB : GV_KSUB, TW = NARROW ? 64 : 128;
  constexpr int UK = MUnit<WE>::UK, PF = MUnit<WE>::PF, KSM = MF_KSP;   // KSM: the X' row stride
  static_assert(!XS || (WE != W_Q4 && XM == X_F16 && UK == 64), "streamed X: q8 / f16 units of 64 k, fp16 X");
  static_assert(GV_NT / 64 * PF * 2048 <= MF_LDS, "X unit slots fit the staging buffer");
  static_assert(KQ * MT * 128 * 4 <= MF_LDS, "partials must fit the staging buffer");
  __shared__ __attribute__((aligned(16))) uint8_t smem[MF_LDS];
  __shared__ uint32_t sLast;
  f16 *sX = (f16 *)smem;                                       // [MT][KSM] X', pair order of the encoding
  f32x2 *sG = (f32x2 *)(smem + MT * KSM * 2);                  // [unit][MT] (G1, G2)
  float *sR = (float *)smem;                                   // after the stream: partials

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ch = NARROW ? 0 : wave / GV_KSUB, sub = NARROW ? wave : wave % GV_KSUB, l16 = lane & 15, kc = lane >> 4;
  const uint32_t tile = blockIdx.x / S, slice = blockIdx.x - tile * S;
  const uint32_t nB = tile * (uint32_t)TW, kb0 = slice * KS;
  const uint32_t nuw = KS / UK / KQ, u0 = sub * nuw;
  auto col = [&](uint32_t j) __attribute__((always_inline)) { return NARROW ? j : tile_col(p, (uint32_t)ch, j); };

  // q4: lane l loads weight row l of the wave's 64 (16 bytes + its scale word, as the one-row stream does) and the
  // wave regroups the unit through its own LDS slot; q8 / f16: per block, this lane's weight row and the byte offsets
  // of its codes and scale in the slice's first unit
  uint32_t *wsw = (uint32_t *)(smem + MF_XG) + wave * 320;     // [64 rows][4 words] then [64] scale words
  uint32_t woff[4], soff[4], rlo[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t r = wrow(p, nB + col(WE == W_Q4 ? (uint32_t)lane : (uint32_t)(16 * i + l16)));
    rlo[i] = r & 1u;
    if constexpr (WE == W_Q4) {
      const uint32_t rec = ((r >> 6) * p.wG + ((p.wk0 + kb0) >> 5)) * 1280u;
      woff[i] = rec + (r & 63u) * 16u;
      soff[i] = rec + 1024u + (r & 63u) * 4u;
    } else if constexpr (WE == W_Q8) {
      const uint32_t rec = ((r >> 6) * p.wG + ((p.wk0 + kb0) >> 6)) * 4224u;
      woff[i] = rec + (r & 63u) * 64u + kc * 16u;
      soff[i] = rec + 4096u + (r & 62u) * 2u;
    } else {
      woff[i] = (r * p.wG + p.wk0 + kb0) * 2u + kc * 32u;
      soff[i] = 0u;
    }
  }
  constexpr uint32_t USTRIDE = WE == W_Q4 ? 1280u : WE == W_Q8 ? 4224u : 128u;

  const srsrc wr = stream_rsrc(p.W);
  // XS: lane l copies row l / 4 (rows past M repeat row M - 1, whose outputs are never stored), 16-byte chunk
  // (l % 4) ^ ((l / 16) % 4) of each 32-k half of the unit; slot: [half][row][chunk] (1 KB halves)
  const uint32_t xslot0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)smem + (uint32_t)wave * (PF * 2048u);
  const uint32_t xcr = (uint32_t)lane >> 2 < p.M ? (uint32_t)lane >> 2 : p.M - 1u, xcc = ((uint32_t)lane & 3u) ^ (((uint32_t)lane >> 4) & 3u);
  const uint8_t *xcp = p.X + ((size_t)xcr * p.ldx + p.kx0 + kb0 + xcc * 8u) * 2u;
  auto load = [&](MUnit<WE> &u, uint32_t unit, int slot = 0) {
    const uint32_t du = unit * USTRIDE;
    if constexpr (XS) {
#pragma unroll
      for (int hh = 0; hh < 2; hh++) {
        const uint32_t m0 = __builtin_amdgcn_readfirstlane(xslot0 + (uint32_t)slot * 2048u + (uint32_t)hh * 1024u);
        const uint8_t *src = xcp + (unit * 64u + (uint32_t)hh * 32u) * 2u;
        asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m0), "v"(src) : "memory");
      }
    }
    if constexpr (WE == W_Q4) {
      u.code = sload128(wr, woff[0] + du);
      u.sm = sload32(wr, soff[0] + du);
    } else {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      if constexpr (WE == W_Q8) {
        u.code[i] = sload128(wr, woff[i] + du);
        u.s[i] = sload32(wr, soff[i] + du);
      } else {                                                 // (two loads: 16 whole 128-byte row pieces)
        u.v[i][0] = sload128(wr, woff[i] + du);
        u.v[i][1] = sload128(wr, woff[i] + du + 16u);
      }
    }
    }
  };

  // the nibble masks, the fp16 exponent and the q8 bias in registers (gfx9 VOP3 takes no literal operands)
  uint32_t mlo = 0x000F000Fu, mhi = 0x00F000F0u, mag = 0x64006400u, m64 = 0x64646464u;
  asm volatile("" : "+v"(mlo), "+v"(mhi), "+v"(mag), "+v"(m64));

  f32x4 acc[4];
#pragma unroll
  for (int i = 0; i < 4; i++) acc[i] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  // A rows past M are not staged: the lanes of those rows AND their (unwritten) LDS words with 0
  const uint32_t am = l16 < (int)p.M ? 0xffffffffu : 0u;
  const u32x4 amask = (u32x4){am, am, am, am};

  // XS: the A fragments of the unit in the slot (lane (kc, l16), MFMA h: X row l16, k = 16 kc + 8 h .. + 7, i.e. half
  // kc / 2, chunk 2 (kc % 2) + h), after its copy has landed (W loads were issued after it; loads complete in order)
  auto compute_xs = [&](const MUnit<WE> &u, int slot, auto W) __attribute__((always_inline)) {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(decltype(W)::value) : "memory");
    f16x8 a[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const uint32_t c = 2u * ((uint32_t)kc & 1u) + (uint32_t)h;
      const u32x4 raw = *(const u32x4 *)(smem + (uint32_t)wave * (PF * 2048u) + (uint32_t)slot * 2048u +
                                         ((uint32_t)kc >> 1) * 1024u + (4u * (uint32_t)l16 + (c ^ (((uint32_t)l16 >> 2) & 3u))) * 16u);
      a[h] = __builtin_bit_cast(f16x8, xperm<WE>(raw));
    }
    if constexpr (WE == W_F16) {
#pragma unroll
      for (int h = 0; h < 2; h++)
#pragma unroll
        for (int i = 0; i < 4; i++)
          acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[h], __builtin_bit_cast(f16x8, u.v[i][h]), acc[i], 0, 0, 0);
    } else if constexpr (WE == W_Q8) {
      // -G1 = -1152 (sum of the unit's x) in every column, from a constant B of -1152
      const f16x8 bneg = __builtin_bit_cast(f16x8, (u32x4){0xE480E480u, 0xE480E480u, 0xE480E480u, 0xE480E480u});
      f32x4 ng1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[0], bneg, (f32x4){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
      ng1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[1], bneg, ng1, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        f32x4 d = ng1;
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const uint32_t x0 = (h ? u.code[i].z : u.code[i].x) ^ 0x80808080u, x1 = (h ? u.code[i].w : u.code[i].y) ^ 0x80808080u;
          const u32x4 bw = (u32x4){perm(m64, x0, 0x04020400u), perm(m64, x0, 0x04030401u), perm(m64, x1, 0x04020400u),
                                   perm(m64, x1, 0x04030401u)};
          d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[h], __builtin_bit_cast(f16x8, bw), d, 0, 0, 0);
        }
        const float sc = (float)__builtin_bit_cast(f16, (uint16_t)(rlo[i] ? (u.s[i] >> 16) : (u.s[i] & 0xffffu)));
#pragma unroll
        for (int r = 0; r < 4; r++) acc[i][r] = fmaf(sc, d[r], acc[i][r]);
      }
    }
  };

  auto compute = [&](const MUnit<WE> &u, uint32_t unit) {
    if constexpr (WE == W_F16) {
      // lane kc holds k 16 kc .. 16 kc + 15 of the unit, 8 of them per MFMA
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const f16x8 a = __builtin_bit_cast(f16x8, *(const u32x4 *)(sX + l16 * KSM + unit * UK + 16 * kc + 8 * h) & amask);
#pragma unroll
        for (int i = 0; i < 4; i++)
          acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(f16x8, u.v[i][h]), acc[i], 0, 0, 0);
      }
    } else {
      // (G1, G2) of rows m = 4 kc + r for this unit
      const f32x4 *gp = (const f32x4 *)(sG + unit * MT + 4 * kc);
      const f32x4 ga = gp[0], gb = gp[1];
      const float g1[4] = {ga.x, ga.z, gb.x, gb.z}, g2[4] = {ga.y, ga.w, gb.y, gb.w};
      // the MFMA starts from -G1, so it returns D - G1 directly
      const f32x4 ng1 = (f32x4){-g1[0], -g1[1], -g1[2], -g1[3]};
      f32x4 d[4];
#pragma unroll
      for (int i = 0; i < 4; i++) d[i] = ng1;
      // q4: regroup the unit inside the wave: lane (kc, l16) takes word kc of row 16 i + l16 and that row's scale
      uint32_t qw[4], qs[4];
      if constexpr (WE == W_Q4) {
        *(u32x4 *)(wsw + 4 * lane) = u.code;
        wsw[256 + lane] = u.sm;
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int i = 0; i < 4; i++) {
          qw[i] = wsw[4 * (16 * i + l16) + kc];
          qs[i] = wsw[256 + 16 * i + l16];
        }
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
      }
#pragma unroll
      for (int h = 0; h < UK / 32; h++) {
        // q8: lane kc holds k 16 kc .. 16 kc + 15 of the unit (one 16-byte load per row), 8 of them per MFMA
        const int ka = WE == W_Q8 ? 16 * kc + 8 * h : 32 * h + 8 * kc;
        const f16x8 a = __builtin_bit_cast(f16x8, *(const u32x4 *)(sX + l16 * KSM + unit * UK + ka) & amask);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          u32x4 bw;
          if constexpr (WE == W_Q4) {
            const uint32_t w = qw[i], w8 = w >> 8;
            bw = (u32x4){(w & mlo) | mag, (w & mhi) | mag, (w8 & mlo) | mag, (w8 & mhi) | mag};
          } else {
            const uint32_t x0 = (h ? u.code[i].z : u.code[i].x) ^ 0x80808080u, x1 = (h ? u.code[i].w : u.code[i].y) ^ 0x80808080u;
            bw = (u32x4){perm(m64, x0, 0x04020400u), perm(m64, x0, 0x04030401u), perm(m64, x1, 0x04020400u),
                         perm(m64, x1, 0x04030401u)};
          }
          d[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(f16x8, bw), d[i], 0, 0, 0);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        float s, mn = 0.0f;
        if constexpr (WE == W_Q4) {
          const f16x2 sm2 = as_h2(qs[i]);
          s = (float)sm2.x; mn = (float)sm2.y;
        } else {
          s = (float)__builtin_bit_cast(f16, (uint16_t)(rlo[i] ? (u.s[i] >> 16) : (u.s[i] & 0xffffu)));
        }
#pragma unroll
        for (int r = 0; r < 4; r++) acc[i][r] = fmaf(s, d[i][r], fmaf(mn, g2[r], acc[i][r]));
      }
    }
  };

  if constexpr (XS) {
    // (every ring entry is loaded, clamped to the wave's last unit, so the loads younger than each unit's copy are
    // counted exactly: LPU weight loads per unit, 2 copies)
    constexpr int LPU = 8;                                     // q8: 4 code + 4 scale loads; f16: 8 code loads
    const uint32_t nl = nuw ? nuw - 1u : 0u;
    MUnit<WE> ring[PF];
#pragma unroll
    for (int j = 0; j < PF; j++) {
      load(ring[j], u0 + ((uint32_t)j < nl ? (uint32_t)j : nl), j);
      __builtin_amdgcn_sched_barrier(0);
    }
    uint32_t j0 = 0;
#pragma unroll 1
    for (; j0 + PF <= nuw; j0 += PF) {
#pragma unroll
      for (int j = 0; j < PF; j++) {
        compute_xs(ring[j], j, std::integral_constant<int, LPU + (PF - 1) * (LPU + 2)>{});
        const uint32_t nx = j0 + PF + j;
        load(ring[j], u0 + (nx < nuw ? nx : nl), j);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    static_assert(PF <= 4, "the tail below covers up to 4 units in flight");
    auto tail = [&](auto J) __attribute__((always_inline)) {
      constexpr int j = decltype(J)::value;
      if constexpr (j < PF)
        if (j0 + j < nuw) compute_xs(ring[j], j, std::integral_constant<int, LPU + (PF - 1 - j) * (LPU + 2)>{});
    };
    tail(std::integral_constant<int, 0>{});
    tail(std::integral_constant<int, 1>{});
    tail(std::integral_constant<int, 2>{});
    tail(std::integral_constant<int, 3>{});
    __builtin_amdgcn_s_waitcnt(0x0f70);                          // vmcnt(0): no copy may land after this
    __syncthreads();                                             // the slots are dead: the buffer takes the partials
  } else {
  // X' of the slice for the rows < M only (the MFMA A reads of rows past M take zeros instead); one thread per
    // (row, unit) task stages the unit's chunks and (q4 / q8) its sums of the unscaled X' over the low / high positions
    // -> (G1, G2); q4: the high-nibble positions (odd pair slots) are stored as x / 16. The chunks of the first XT
    // tasks of every thread (all of them for K <= 4096 and 16 rows) are loaded before the ring: loads return in issue
    // order, so X loaded behind the ring would wait for its HBM units, with the ring then idle until the staging ends.
    constexpr int CPT = UK / 8, XT = 16 / CPT;
    const uint32_t ng = KS / UK, Mr = p.M < (uint32_t)MT ? p.M : (uint32_t)MT, ntask = Mr * ng;
    u32x4 xr[XT][CPT];
  #pragma unroll
    for (int i = 0; i < XT; i++) {
      const uint32_t t = tid + i * GV_NT, m = t / ng, g = t - m * ng;
  #pragma unroll
      for (int q = 0; q < CPT; q++)
        xr[i][q] = t < ntask ? xload8<XM>(p, m, RowCtx{0, 0, 0}, kb0 + g * UK + 8 * q) : (u32x4){0u, 0u, 0u, 0u};
    }
    __builtin_amdgcn_sched_barrier(0);
  
    MUnit<WE> ring[PF];
  #pragma unroll
    for (int j = 0; j < PF; j++)
      if ((uint32_t)j < nuw) load(ring[j], u0 + j);
    __builtin_amdgcn_sched_barrier(0);
  
    const f16x2 r16 = {(f16)0.0625f, (f16)0.0625f};
    auto stage = [&](uint32_t t, const u32x4 *xin) __attribute__((always_inline)) {
      const uint32_t m = t / ng, g = t - m * ng;
      float lo = 0.0f, hi = 0.0f;
  #pragma unroll
      for (int q = 0; q < CPT; q++) {
        u32x4 xv = xperm<WE>(xin[q]);
        if constexpr (WE != W_F16) {
          const f16x2 a = as_h2(xv.x), b = as_h2(xv.y), c = as_h2(xv.z), d = as_h2(xv.w);
          lo += ((float)a.x + (float)a.y) + ((float)c.x + (float)c.y);
          hi += ((float)b.x + (float)b.y) + ((float)d.x + (float)d.y);
          if constexpr (WE == W_Q4) {
            xv.y = as_u(b * r16);
            xv.w = as_u(d * r16);
          }
        }
        *(u32x4 *)(sX + m * KSM + g * UK + 8 * q) = xv;
      }
      if constexpr (WE == W_Q4) sG[g * MT + m] = (f32x2){1024.0f * lo + 64.0f * hi, lo + hi};
      else if constexpr (WE == W_Q8) sG[g * MT + m] = (f32x2){1152.0f * (lo + hi), 0.0f};
    };
  #pragma unroll
    for (int i = 0; i < XT; i++) {
      const uint32_t t = tid + i * GV_NT;
      if (t < ntask) stage(t, xr[i]);
    }
    for (uint32_t t = tid + XT * GV_NT; t < ntask; t += GV_NT) {
      u32x4 xin[CPT];
      const uint32_t m = t / ng, g = t - m * ng;
  #pragma unroll
      for (int q = 0; q < CPT; q++) xin[q] = xload8<XM>(p, m, RowCtx{0, 0, 0}, kb0 + g * UK + 8 * q);
      stage(t, xin);
    }
    __syncthreads();
  
    uint32_t j0 = 0;
  #pragma unroll 1
    for (; j0 + PF <= nuw; j0 += PF) {
  #pragma unroll
      for (int j = 0; j < PF; j++) {
        compute(ring[j], u0 + j0 + j);
        const uint32_t nx = j0 + PF + j;
        load(ring[j], u0 + (nx < nuw ? nx : nuw - 1u));
      }
    }
  #pragma unroll
    for (int j = 0; j < PF; j++)
      if (j0 + j < nuw) compute(ring[j], u0 + j0 + j);
    __syncthreads();                                             // X' is dead: the buffer takes the partials
  
  }

  // D[m = 4 kc + r][row 16 i + l16]
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int r = 0; r < 4; r++) sR[(sub * MT + 4 * kc + r) * 128 + col((uint32_t)(16 * i + l16))] = acc[i][r];
  __syncthreads();
  if constexpr (NARROW) finish_fast<MT, KQ, GV_NT, TW>(p, sR, nB, tid);     // (the host sends only S = 1 here)
  else if (fast_epi(p, S)) finish_fast<MT>(p, sR, nB, tid);
  else finish<MT>(p, sR, part, cnt, S, tile, slice, nB, tid, &sLast);
}

// ------------------------------------------------------------------------------------------------------------------
// Decode on the matrix cores with q4 weights and 5..16 rows (3..16 with the stream kernel's matrix-core form switched
// off), with no X' staging phase before the stream (the X rows
// are copied to LDS while the first weight units are on their way). The same 128-column items as above,
// but each of the 8 waves covers all 128 columns of one K-eighth, so each X' fragment it loads serves 8 blocks of 16
// weight rows. Per 32-k unit a wave runs ten v_mfma_f32_16x16x32_f16, every operand in registers:
//   * lane l loads code row l of each of the item's two 64-row halves (tile_col; 16 bytes each: one 128-bit load covers
//     64 rows' 1 KB) and their
//     (scale, min) words, as the one-row stream does; a 4 x 4 transpose across the four 16-lane groups (two
//     v_permlane32_swap and two v_permlane16_swap per 64 rows) then gives lane (kc = l / 16, l16 = l % 16) code word
//     kc of row 16 i + l16 in register i, the B fragment of block i (magic-biased in place: 1024 + q low nibbles,
//     1024 + 16 q high), and the same swaps broadcast row 16 i + l16's (scale, min) word to it
//   * each lane reads its A fragment, X' row l16 (rows past M repeat row M - 1, whose products land in output rows
//     that are never stored), k = 8 kc .. 8 kc + 7 of the unit, and puts it into the pair order of the decode, the
//     high-nibble positions scaled by 1/16. fp16 X with 16-byte rows (XL): each unit's 16 X rows x 32 k (1 KB) are
//     copied to the wave's LDS slot of its ring entry by one load-to-LDS instruction (global_load_lds_dwordx4, no
//     registers) issued with the unit's weight loads, so X streams with the weights instead of being staged whole
//     before them (16 rows x 4096 k: 128 KB per item, 18.7-19.1 against 19.8-19.9 us at M = 16). Otherwise (rms / lnmod prologues, unaligned X) the fragment is computed from X with
//     the same unit's loads.
//   * two MFMAs against constant B operands give, for every output column, -G1 = -(1024 X_lo + 64 X_hi) and
//     G2 = X_lo + X_hi of the unit's rows; each block's MFMA starts from -G1, so it returns sum x q directly, and
//     y += s (sum x q) + mn G2 in registers (the fp32 weight model of the stream above).
// (12 or 16 waves per item measured slower; with X streamed per unit, 2 units in flight per wave beat 1, 3 and 4:
// M = 16 17.7-18.1 against 18.3-18.4 / 18.2-18.5 / 19.8-19.9 us, M = 8 16.8-17.2 against 17.9 / 17.3-17.8 / 18.4)
#ifndef P0K_MQ_PF
#define P0K_MQ_PF 2
#endif
constexpr int MQ_KQ = 8, MQ_NT = 64 * MQ_KQ, MQ_PF = P0K_MQ_PF;     // waves = K parts of an item; units in flight per wave
// NARROW: items of 64 ws columns (one half: 4 blocks of 16 rows), S = 1 and the element-wise epilogues only, for calls
// whose 128-column items the planner would split (the same rule as the one-row stream's 64-column items)
template <int XM, bool XL, bool NARROW = false>
__global__ __launch_bounds__(MQ_NT) void k_gemv_mq4(Params p, float *part, uint32_t *cnt, uint32_t S, uint32_t KS) {
  constexpr int MT = 16, PF = MQ_PF, NH = NARROW ? 1 : 2, TW = 64 * NH;   // halves (64-row blocks) per item
  static_assert(!XL || XM == X_F16, "X rows are copied as they are only without a prologue");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[MQ_KQ * MT * 128 * 4];
  static_assert(MQ_KQ * MQ_PF * 1024 <= MQ_KQ * MT * 128 * 4, "X unit slots fit the partials' buffer");
  __shared__ uint32_t sLast;
  float *sR = (float *)smem;                                   // after the stream: the K-eighths' partials

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, kc = lane >> 4;
  const uint32_t tile = blockIdx.x / S, slice = blockIdx.x - tile * S;
  const uint32_t nB = tile * (uint32_t)TW, kb0 = slice * KS;
  const uint32_t nu = KS / 32u, u0 = wave * nu / MQ_KQ, nuw = (wave + 1) * nu / MQ_KQ - u0;   // units of this wave

  // this lane's weight rows (lane and 64 + lane of the tile): byte offsets of their code rows and (scale, min) words in
  // the wave's first unit (32-bit: tensors of 4 GiB or more take the MFMA GEMM)
  uint32_t woff[NH], soff[NH];
#pragma unroll
  for (int h = 0; h < NH; h++) {
    const uint32_t r = wrow(p, nB + (NARROW ? (uint32_t)lane : tile_col(p, (uint32_t)h, (uint32_t)lane)));
    const uint32_t rec = ((r >> 6) * p.wG + ((p.wk0 + kb0) >> 5) + u0) * 1280u;
    woff[h] = rec + (r & 63u) * 16u;
    soff[h] = rec + 1024u + (r & 63u) * 4u;
  }
  const uint32_t xrow = (uint32_t)l16 < p.M ? (uint32_t)l16 : p.M - 1u;
  const uint32_t xk0 = kb0 + u0 * 32u + (uint32_t)kc * 8u;

  // XL: the unit's X' block (16 rows x 32 k, 1 KB) goes to this wave's LDS slot for the ring entry by one load-to-LDS
  // instruction issued with the unit's weight loads (before them, so it has landed once they have): lane l copies row
  // l / 4, 16-byte chunk (l % 4) ^ ((l / 16) % 4) of it (rows past M repeat row M - 1); the chunk swizzle makes the
  // A reads (lane (kc, l16): row l16, chunk kc) conflict-free
  const uint32_t xslot0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)smem + (uint32_t)wave * (MQ_PF * 1024u);
  const uint32_t xcr = (uint32_t)lane >> 2 < p.M ? (uint32_t)lane >> 2 : p.M - 1u, xcc = ((uint32_t)lane & 3u) ^ (((uint32_t)lane >> 4) & 3u);
  const uint8_t *xcp = p.X + ((size_t)xcr * p.ldx + p.kx0 + kb0 + u0 * 32u + xcc * 8u) * 2u;
  const uint32_t xrd = (uint32_t)wave * (MQ_PF * 1024u) + (4u * (uint32_t)l16 + ((uint32_t)kc ^ (((uint32_t)l16 >> 2) & 3u))) * 16u;

  struct U { u32x4 code[NH]; uint32_t sm[NH]; u32x4 x; };
  const srsrc wr = stream_rsrc(p.W);
  auto load = [&](U &u, uint32_t j, int slot) __attribute__((always_inline)) {
    const uint32_t du = j * 1280u;
    if constexpr (XL) {
      const uint32_t m0 = __builtin_amdgcn_readfirstlane(xslot0 + (uint32_t)slot * 1024u);
      const uint8_t *src = xcp + j * 64u;
      asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m0), "v"(src) : "memory");
    }
#pragma unroll
    for (int h = 0; h < NH; h++) u.code[h] = sload128(wr, woff[h] + du);
#pragma unroll
    for (int h = 0; h < NH; h++) u.sm[h] = sload32(wr, soff[h] + du);
    if constexpr (!XL) u.x = xload8<XM>(p, xrow, RowCtx{0, 0, 0}, xk0 + j * 32u);
  };
  // the A fragment of the wave's unit j
  auto xfrag = [&](const U &u, int slot) __attribute__((always_inline)) -> u32x4 {
    if constexpr (XL) return *(const u32x4 *)(smem + xrd + (uint32_t)slot * 1024u);
    else return u.x;
  };

  uint32_t mlo = 0x000F000Fu, mhi = 0x00F000F0u, mag = 0x64006400u;
  asm volatile("" : "+v"(mlo), "+v"(mhi), "+v"(mag));
  // B of -G1: every half -1024; B of G2: 1 at the low-nibble positions (pair slots 0, 2), 16 at the high ones (1, 3)
  const f16x8 bneg = __builtin_bit_cast(f16x8, (u32x4){0xE400E400u, 0xE400E400u, 0xE400E400u, 0xE400E400u});
  const f16x8 bg2 = __builtin_bit_cast(f16x8, (u32x4){0x3C003C00u, 0x4C004C00u, 0x3C003C00u, 0x4C004C00u});
  const f16x2 r16 = {(f16)0.0625f, (f16)0.0625f};
  const f32x4 z4 = {0.0f, 0.0f, 0.0f, 0.0f};

  f32x4 acc[4 * NH];
#pragma unroll
  for (int i = 0; i < 4 * NH; i++) acc[i] = z4;

  // XL: before the unit's X' read, wait for its copy: W loads were issued after it (own weights, then the other
  // entries of the ring), and loads complete in order
  auto compute = [&](const U &u, int slot, auto W) __attribute__((always_inline)) {
    if constexpr (XL) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(decltype(W)::value) : "memory");
    u32x4 xv = xperm<W_Q4>(xfrag(u, slot));
    xv.y = as_u(as_h2(xv.y) * r16);
    xv.w = as_u(as_h2(xv.w) * r16);
    const f16x8 a = __builtin_bit_cast(f16x8, xv);
    const f32x4 ng1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bneg, z4, 0, 0, 0);
    const f32x4 g2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bg2, z4, 0, 0, 0);
#pragma unroll
    for (int h = 0; h < NH; h++) {
      // the 4 x 4 transpose of (16-lane group, code word): word kc of row 64 h + 16 i + l16 into register i
      uint32_t w[4];
      {
        const auto p02 = __builtin_amdgcn_permlane32_swap(u.code[h].x, u.code[h].z, false, false);
        const auto p13 = __builtin_amdgcn_permlane32_swap(u.code[h].y, u.code[h].w, false, false);
        const auto q01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
        const auto q23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
        w[0] = q01[0]; w[1] = q01[1]; w[2] = q23[0]; w[3] = q23[1];
      }
      // row 64 h + 16 i + l16's (scale, min) word, from lane 16 i + l16, into register i
      uint32_t sm[4];
      {
        const auto t = __builtin_amdgcn_permlane32_swap(u.sm[h], u.sm[h], false, false);
        const auto q0 = __builtin_amdgcn_permlane16_swap(t[0], t[0], false, false);
        const auto q1 = __builtin_amdgcn_permlane16_swap(t[1], t[1], false, false);
        sm[0] = q0[0]; sm[1] = q0[1]; sm[2] = q1[0]; sm[3] = q1[1];
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t w8 = w[i] >> 8;
        const u32x4 bw = (u32x4){(w[i] & mlo) | mag, (w[i] & mhi) | mag, (w8 & mlo) | mag, (w8 & mhi) | mag};
        const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(f16x8, bw), ng1, 0, 0, 0);
        const f16x2 sm2 = as_h2(sm[i]);
        const float s = (float)sm2.x, mn = (float)sm2.y;
#pragma unroll
        for (int r = 0; r < 4; r++) acc[4 * h + i][r] = fmaf(s, d[r], fmaf(mn, g2[r], acc[4 * h + i][r]));
      }
    }
  };

  // (a slice shorter than 8 units leaves waves idle; their ring loads stay inside the item's first unit)
  const uint32_t nl = nuw ? nuw - 1u : 0u;
  U ring[PF];
#pragma unroll
  for (int j = 0; j < PF; j++) {
    load(ring[j], (uint32_t)j < nl ? (uint32_t)j : nl, j);
    __builtin_amdgcn_sched_barrier(0);
  }
  uint32_t j0 = 0;
#pragma unroll 1
  for (; j0 + PF <= nuw; j0 += PF) {
    constexpr int LPU = 2 * NH;                                // weight loads per unit
#pragma unroll
    for (int j = 0; j < PF; j++) {
      compute(ring[j], j, std::integral_constant<int, LPU + (PF - 1) * (LPU + 1)>{});
      const uint32_t nx = j0 + PF + j;
      load(ring[j], nx < nuw ? nx : nl, j);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // (the tail issues no loads: fewer are younger than each unit's copy)
  constexpr int LPU = 2 * NH;
  static_assert(PF >= 1 && PF <= 4, "the tail below covers 1..4 units in flight");
  auto tail = [&](auto J) __attribute__((always_inline)) {
    constexpr int j = decltype(J)::value;
    if constexpr (j < PF)
      if (j0 + j < nuw) compute(ring[j], j, std::integral_constant<int, LPU + (PF - 1 - j) * (LPU + 1)>{});
  };
  tail(std::integral_constant<int, 0>{});
  tail(std::integral_constant<int, 1>{});
  tail(std::integral_constant<int, 2>{});
  tail(std::integral_constant<int, 3>{});
  if constexpr (XL) {                                          // the X' slots are dead: the buffer takes the partials
    __builtin_amdgcn_s_waitcnt(0x0f70);                        // vmcnt(0): no copy may land after this
    __syncthreads();
  }

  // D[m = 4 kc + r][row 16 i + l16] of the tile's rows 64 h + ...; the K-eighths meet in LDS
#pragma unroll
  for (int i = 0; i < 4 * NH; i++)
#pragma unroll
    for (int r = 0; r < 4; r++)
      sR[(wave * MT + 4 * kc + r) * 128 +
         (NARROW ? (uint32_t)(16 * i + l16) : tile_col(p, (uint32_t)(i >> 2), (uint32_t)(16 * (i & 3) + l16)))] = acc[i][r];
  __syncthreads();
  if constexpr (NARROW) finish_fast<MT, MQ_KQ, MQ_NT, TW>(p, sR, nB, tid);   // (the host sends only S = 1 here)
  else if (fast_epi(p, S)) finish_fast<MT, MQ_KQ, MQ_NT>(p, sR, nB, tid);
  else finish<MT, MQ_KQ, MQ_NT>(p, sR, part, cnt, S, tile, slice, nB, tid, &sLast);
}

// the row tile of the stream kernel: q4 with mx takes the matrix-core form (4 rows) at M = 2 too
static uint32_t stream_mt(uint32_t M, int we, bool mx) {
  return M <= 1 ? 1u : (M <= 2 && !(we == W_Q4 && mx)) ? 2u : M <= 4 ? 4u : M <= 8 ? 8u : 16u;
}
template <int MT>
static uint32_t stream_ksm(int we) { return we == W_Q4 && gv_mx<W_Q4, MT>() ? (uint32_t)mx_ksm<MT>() : (uint32_t)ks_max<MT>(); }
static uint32_t ks_max_of(uint32_t M, int we, bool mf, bool mx) {
  if (mf) return MF_KSM;
  switch (stream_mt(M, we, mx)) {
  case 1: return stream_ksm<1>(we);
  case 2: return stream_ksm<2>(we);
  case 4: return stream_ksm<4>(we);
  case 8: return stream_ksm<8>(we);
  }
  return stream_ksm<16>(we);
}
unsigned gemv_ks_max(unsigned M, int we, bool mf, bool mx) { return ks_max_of(M, we, mf, mx); }
// k of one weight unit: q8 64 (a record), f16 on the matrix cores 64 (one 128-byte row piece), else 32
unsigned gemv_unit_k(int we, bool mf) { return we == W_Q8 || (we == W_F16 && mf) ? 64u : 32u; }

// Slices per tile: the fewest that fill the GPU with items (about one per CU) and keep each slice's X' inside the LDS
// budget, with a whole number of units per K-quarter.
void gemv_split(const Params &p, int we, unsigned cus, bool mf, bool mx, unsigned *S_out, unsigned *KS_out) {
  const uint32_t tiles = (p.N + 127) / 128;
  const uint32_t quant = gemv_unit_k(we, mf) * GV_KSUB;     // k per "one unit in each K-quarter"
  const uint32_t ksm = ks_max_of(p.M, we, mf, mx);
  uint32_t S = 1;
  while ((tiles * S < cus * 7u / 8u || p.K / S > ksm) && p.K % (2u * S * quant) == 0) S *= 2u;
  if (p.K % (S * quant) != 0 || p.K / S > ksm) S = 0;             // caller falls back to the MFMA kernel
  *S_out = S;
  *KS_out = S ? p.K / S : 0;
}

template <int WE, int XM, int MT>
static hipError_t launch3(const Params &p, float *part, uint32_t *cnt, uint32_t S, uint32_t KS, hipStream_t s,
                          bool narrow) {
  if (KS > (uint32_t)(gv_mx<WE, MT>() ? mx_ksm<MT>() : ks_max<MT>())) return hipErrorInvalidValue;
  if constexpr (WE == W_Q4 && MT <= 4) {
    if (narrow) {
      if (S != 1 || p.epi == E_HEADS || p.epi == E_ONORMGATE) return hipErrorInvalidValue;
      hipLaunchKernelGGL((k_gemv<WE, XM, MT, true>), dim3((p.N + 63) / 64), dim3(GV_NT), 0, s, p, part, cnt, S, KS);
      return hipGetLastError();
    }
  }
  if (narrow) return hipErrorInvalidValue;
  dim3 grid(((p.N + 127) / 128) * S);
  hipLaunchKernelGGL((k_gemv<WE, XM, MT>), grid, dim3(GV_NT), 0, s, p, part, cnt, S, KS);
  return hipGetLastError();
}
template <int WE, int XM>
static hipError_t launch2(const Params &p, float *part, uint32_t *cnt, uint32_t S, uint32_t KS, hipStream_t s, bool mf,
                          bool mq4, bool mx, bool narrow) {
  if (mf) {
    if (KS > (uint32_t)MF_KSM) return hipErrorInvalidValue;
    dim3 grid(((p.N + 127) / 128) * S);
    if (WE == W_Q4 && mq4) {
      if (narrow) {
        if (S != 1 || p.epi == E_HEADS || p.epi == E_ONORMGATE) return hipErrorInvalidValue;
        const dim3 g64((p.N + 63) / 64);
        if (XM == X_F16 && (p.flags & F_XALIGN8)) hipLaunchKernelGGL((k_gemv_mq4<X_F16, true, true>), g64, dim3(MQ_NT), 0, s, p, part, cnt, S, KS);
        else hipLaunchKernelGGL((k_gemv_mq4<XM, false, true>), g64, dim3(MQ_NT), 0, s, p, part, cnt, S, KS);
        return hipGetLastError();
      }
      if (XM == X_F16 && (p.flags & F_XALIGN8)) hipLaunchKernelGGL((k_gemv_mq4<X_F16, true>), grid, dim3(MQ_NT), 0, s, p, part, cnt, S, KS);
      else hipLaunchKernelGGL((k_gemv_mq4<XM, false>), grid, dim3(MQ_NT), 0, s, p, part, cnt, S, KS);
      return hipGetLastError();
    }
    if (narrow) {
      if (S != 1 || p.epi == E_HEADS || p.epi == E_ONORMGATE) return hipErrorInvalidValue;
      if (WE != W_Q4 && XM == X_F16 && (p.flags & F_XALIGN8) && KS / 64u / (2u * GV_KSUB) >= (uint32_t)MUnit<WE>::PF)
        hipLaunchKernelGGL((k_gemv_mf<WE, XM, true, WE != W_Q4 && XM == X_F16>), dim3((p.N + 63) / 64), dim3(GV_NT), 0, s, p, part, cnt, S, KS);
      else hipLaunchKernelGGL((k_gemv_mf<WE, XM, true>), dim3((p.N + 63) / 64), dim3(GV_NT), 0, s, p, part, cnt, S, KS);
      return hipGetLastError();
    }
    // (streamed X when every ring entry of a wave holds one of its units: the ring is filled unconditionally, so a
    // shorter stream would load its last unit again per empty entry; f16 N 4096 K 2048 in 8 slices, one unit per
    // wave: 15.3 us streamed against 11.5 staged)
    if (WE != W_Q4 && XM == X_F16 && (p.flags & F_XALIGN8) && KS / 64u / GV_KSUB >= (uint32_t)MUnit<WE>::PF)
      hipLaunchKernelGGL((k_gemv_mf<WE, XM, false, WE != W_Q4 && XM == X_F16>), grid, dim3(GV_NT), 0, s, p, part, cnt, S, KS);
    else hipLaunchKernelGGL((k_gemv_mf<WE, XM>), grid, dim3(GV_NT), 0, s, p, part, cnt, S, KS);
    return hipGetLastError();
  }
  switch (stream_mt(p.M, WE, mx)) {
  case 1: return launch3<WE, XM, 1>(p, part, cnt, S, KS, s, narrow);
  case 2: return launch3<WE, XM, 2>(p, part, cnt, S, KS, s, narrow);
  case 4: return launch3<WE, XM, 4>(p, part, cnt, S, KS, s, narrow);
  case 8: return launch3<WE, XM, 8>(p, part, cnt, S, KS, s, narrow);
  }
  return launch3<WE, XM, 16>(p, part, cnt, S, KS, s, narrow);
}
template <int WE>
static hipError_t launch1(const Params &p, int xm, float *part, uint32_t *cnt, uint32_t S, uint32_t KS, hipStream_t s,
                          bool mf, bool mq4, bool mx, bool narrow) {
  switch (xm) {
  case X_F16: return launch2<WE, X_F16>(p, part, cnt, S, KS, s, mf, mq4, mx, narrow);
  case X_LNMOD: return launch2<WE, X_LNMOD>(p, part, cnt, S, KS, s, mf, mq4, mx, narrow);
  case X_RMS: return launch2<WE, X_RMS>(p, part, cnt, S, KS, s, mf, mq4, mx, narrow);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemv(const Params &p, int we, int xm, float *part, uint32_t *cnt, uint32_t S, uint32_t KS,
                       hipStream_t s, bool mf, bool mq4, bool mx, bool narrow) {
  const uint32_t quant = gemv_unit_k(we, mf) * GV_KSUB;
  if (p.M > (uint32_t)GEMV_MAX_M || S == 0 || KS * S != p.K || KS % quant) return hipErrorInvalidValue;
  if (narrow && (S != 1 || KS % (2 * quant) || (!mf && we != W_Q4))) return hipErrorInvalidValue;
  switch (we) {
  case W_Q4: return launch1<W_Q4>(p, xm, part, cnt, S, KS, s, mf, mq4, mx, narrow);
  case W_Q8: return launch1<W_Q8>(p, xm, part, cnt, S, KS, s, mf, mq4, mx, narrow);
  case W_F16: return launch1<W_F16>(p, xm, part, cnt, S, KS, s, mf, mq4, mx, narrow);
  }
  return hipErrorInvalidValue;
}

}  // namespace p0k
