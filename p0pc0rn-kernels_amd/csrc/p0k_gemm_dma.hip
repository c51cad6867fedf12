// p0k_gemm_dma.hip — the prefill path of `gemm` (src/ops/gemm.js:29-257) for row-major fp16 activations: operands
// move global -> LDS by the load-to-LDS path (global_load_lds_dwordx4 / _dword: each lane's bytes land at
// M0 + 16 lane / 4 lane, no registers, no LDS store instructions), weights are decoded in registers right before the
// matrix core uses them.
//
// One workgroup computes a TBM x TBN tile (TBM, TBN in {128, 256}): 4 waves (2 x 2) for the smaller tiles, 8 waves
// (2 x 4, two per SIMD, so one wave's decode and LDS reads run under the other's MFMAs) for 256 x 256 and, with f16
// or q8 weights, 256 x 128; a wave owns (TBM/2) x (TBN/2), 128 x 64 or 128 x 32 as 32x32 v_mfma_f32_32x32x16_f16
// blocks. K moves in steps of 64 through a ring of S LDS stages:
//   X' rows      [row][128 B], the 16-byte chunk c of row r at c ^ ((r >> 1) & 7)
//   f16 weights  the same layout, one row per ws column
//   q4 records   per 64-column block and 32-k record: the 64 code rows [col][16 B] as stored, and the 64 (scale, min)
//                words [col][4 B]; q8 records: the code rows as four 16-byte chunks [chunk][col][16 B] and the scale
//                words [col][4 B] (the word holding the row's fp16 scale)
// Column `col` of the tile reads weight row wrow(col) (GLU interleave and clamping in wrow), so one DMA instruction
// gathers 64 columns' records in place. A step is four 16-k sub-steps; lane l takes A row l % 32 and B column l % 32
// of its blocks and k = 32 h + 8 s .. + 7 (h = l / 32, s = sub-step): the 8 codes of ONE q4 code word (word s of
// record h), half of one q8 16-byte chunk, one f16 chunk. Decoding follows p0k_device.h bit for bit in value (the q4
// odd nibble is read in place as the fp16 1024 + 16 q and scaled by s / 16, exact because s / 16 is a normal fp16
// whenever the fast path is taken), in natural k order, so X' needs no permutation.
//
// Pipeline (per wave): the sub-step's MFMAs are interleaved with the LDS reads of the next sub-step's X' fragments,
// the decode of its weight fragments and one third of the DMA refill of the stage freed at the last barrier. One
// barrier per step: before it, s_waitcnt vmcnt(n) leaves only the refills younger than the next stage in flight; the
// DMA instructions are invisible to the compiler (inline asm), so every wait on them is explicit and exact.
// After the last step the fp32 accumulators go through LDS in 128 x 128 quadrants to the shared epilogue. The K
// order of every output element is fixed (no split-K) and independent of the tile.
#include "p0k_device.h"
#include "p0k_launch.h"

#include <type_traits>

namespace p0k {

namespace {

constexpr int DBK = 64;

// NWV waves laid out WGM x (NWV / WGM): 4 as 2 x 2, 8 as 2 x 4 (two waves per SIMD), or 4 as 1 x 4 (WGM = 1: one
// wave per SIMD, each over all TBM rows, so a decoded weight fragment feeds TBM / 32 MFMAs)
template <int WE, int TBM, int TBN, int NWV = 4, int WGM = 2>
struct DT {
  static constexpr int NT = 64 * NWV;
  static constexpr int NBLK = TBN / 64;                                        // 64-column weight blocks
  // DMA instructions per stage, in groups of NWV (one per wave): X' row blocks (8 rows), weight code blocks, then
  // weight scale words (q8: padded to NWV with repeats of the last block's)
  static constexpr int NIA = TBM / 8;
  static constexpr int NIC = WE == W_F16 ? TBN / 8 : (WE == W_Q4 ? NBLK * 2 : NBLK * 4);
  static constexpr int NIS = WE == W_F16 ? 0 : (WE == W_Q4 ? NBLK * 2 : NWV);
  // the A instructions split evenly over the waves; the weight code and scale instructions together (a wave's one
  // instruction may then be a code block for some waves and a scale block for others: q4 256 x 128 with 8 waves)
  static_assert(NIA % NWV == 0 && (NIC + NIS) % NWV == 0, "DMA instructions per wave");
  static constexpr bool WSPLIT = NIC % NWV == 0;                               // codes / scales on whole rounds
  static constexpr int NW = (NIA + NIC + NIS) / NWV;                           // per wave
  static constexpr int WA = NIA / NWV, WC = NIC / NWV;
  static constexpr int A_BYTES = TBM * 128;
  static constexpr int BC_BYTES = WE == W_F16 ? TBN * 128 : (WE == W_Q4 ? NBLK * 2 * 1024 : NBLK * 4 * 1024);
  static constexpr int BS_BYTES = NIS * 256;
  static constexpr int STAGE = A_BYTES + BC_BYTES + BS_BYTES;
  static constexpr bool TWO = NWV == 4 && WGM == 2 && 4 * STAGE <= 160 * 1024 && TBM * TBN < 256 * 256;  // two WGs per CU
  static constexpr int BUDGET = TWO ? 80 * 1024 : 160 * 1024;
  static constexpr int S = 3 * STAGE <= BUDGET ? 3 : 2;
  // the epilogue's fp32 staging: with one workgroup per CU the whole LDS is free after the K loop, so 128 rows of the
  // full tile width (or the whole 256 x 128 tile) go through it at once; two workgroups per CU keep 128 x 128 quadrants
  static constexpr bool WIDE = !TWO;
  static constexpr int CW = WIDE ? TBN : 128, CR = WIDE ? (TBN == 128 ? TBM : 128) : 128, CLD = CW + 4;
  static constexpr int SMEM_C = CR * CLD * 4;
  static constexpr int SMEM = S * STAGE > SMEM_C ? S * STAGE : SMEM_C;
  static_assert(SMEM <= BUDGET, "LDS budget");
  static constexpr int WGN = NWV / WGM;                                        // waves along N
  static constexpr int WTM = TBM / WGM, WTN = TBN / WGN;                       // a wave's sub-tile
  static constexpr int BI = WTM / 32, BJ = WTN / 32;                           // 32x32 blocks per wave
  static constexpr int WGS = TWO ? 2 : 1;                                      // workgroups per CU
  static constexpr int OCC = WGS * NWV / 4;                                    // waves per SIMD
};

__device__ __forceinline__ uint32_t lds_u32(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
// load-to-LDS of 16 (4) bytes per lane from the uniform base + the lane's 32-bit offset: lane l writes LDS
// [m0 + 16 l] ([m0 + 4 l])
// a wave-uniform pointer in SGPRs (the "s" constraint does not move a value the compiler keeps in VGPRs)
__device__ __forceinline__ const uint8_t *sgpr_ptr(const uint8_t *p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const uint8_t *)(uintptr_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ void dma16(const uint8_t *base, uint32_t off, uint32_t m0) {
  base = sgpr_ptr(base);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(m0), "v"(off), "s"(base) : "memory");
}
__device__ __forceinline__ void dma16a(const uint8_t *addr, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m0), "v"(addr) : "memory");
}
__device__ __forceinline__ void dma4(const uint8_t *base, uint32_t off, uint32_t m0) {
  base = sgpr_ptr(base);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(m0), "v"(off), "s"(base) : "memory");
}
// s_waitcnt vmcnt(n) alone (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[15:14])
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xc07f); }
__device__ __forceinline__ void stage_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// q4: the (scale, min) word allows the fast decode (p0k_device.h) and s / 16 is exact
__device__ __forceinline__ bool q4n_fast_ok(uint32_t sm) {
  const uint32_t es = (sm >> 10) & 31u;
  return q4_fast_ok(sm) && (es >= 5u || (sm & 0x7fffu) == 0u);
}
// q4 code word (k0..k7, low nibble first) -> f16x8 in natural order
// (msk, mag: 0x00F0000F and 0x64006400 held in registers, so the mask-and-bias is one v_and_or_b32)
__device__ __forceinline__ f16x8 dq4_fast(uint32_t w, f16x2 s2, f16x2 m2, uint32_t msk, uint32_t mag) {
  const f16x2 k1024 = {(f16)1024.0f, (f16)1024.0f};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    // byte i to bytes 0 and 2: (q_2i | 16 q_2i+1) in both halves; the mask keeps q_2i low, 16 q_2i+1 high
    const uint32_t t = perm(w, w, 0x0c000c00u | (uint32_t)i | ((uint32_t)i << 16));
    const uint32_t v = (t & msk) | mag;
    o[i] = as_u(__builtin_elementwise_fma(as_h2(v) - k1024, s2, m2));
  }
  return __builtin_bit_cast(f16x8, (u32x4){o[0], o[1], o[2], o[3]});
}
__device__ __forceinline__ f16x8 dq4_slow(uint32_t w, uint32_t sm) {
  const f16x2 sm2 = as_h2(sm);
  const float s = (float)sm2.x, mn = (float)sm2.y;
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    float a = fmaf((float)((w >> (8 * i)) & 15u), s, mn), b = fmaf((float)((w >> (8 * i + 4)) & 15u), s, mn);
    asm volatile("" : "+v"(a), "+v"(b));   // fp32 rounding first, as the reference (no fused fma + cvt)
    o[i] = as_u((f16x2){(f16)a, (f16)b});
  }
  return __builtin_bit_cast(f16x8, (u32x4){o[0], o[1], o[2], o[3]});
}
// q8: two code words (k0..k7 as signed bytes) -> f16x8 natural order, f16(q * s)
__device__ __forceinline__ f16x8 dq8(uint32_t w0, uint32_t w1, f16x2 s2) {
  const f16x2 k1152 = {(f16)1152.0f, (f16)1152.0f};
  const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
  const uint32_t o0 = as_u((as_h2(perm(0x64646464u, u0, 0x04010400u)) - k1152) * s2);
  const uint32_t o1 = as_u((as_h2(perm(0x64646464u, u0, 0x04030402u)) - k1152) * s2);
  const uint32_t o2 = as_u((as_h2(perm(0x64646464u, u1, 0x04010400u)) - k1152) * s2);
  const uint32_t o3 = as_u((as_h2(perm(0x64646464u, u1, 0x04030402u)) - k1152) * s2);
  return __builtin_bit_cast(f16x8, (u32x4){o0, o1, o2, o3});
}

__device__ __forceinline__ void tile_order(const Params &p, uint32_t bid, uint32_t &mt, uint32_t &nt) {
  // consecutive workgroups go to different XCDs: regroup per XCD, then walk bands of 4 M-tiles (shared L2 rows; with
  // q8 2048 x 4096 in one round an XCD then holds 4 M-tiles x 8 N-tiles of operands instead of 8 x 4: 2% faster)
  const uint32_t total = p.tilesM * p.tilesN;
  uint32_t t = bid;
  if ((total & 7u) == 0u) t = (bid & 7u) * (total >> 3) + (bid >> 3);
  const uint32_t band = 4u, per = band * p.tilesN, g = t / per, first = g * band;
  const uint32_t rows = p.tilesM - first < band ? p.tilesM - first : band, in = t - g * per;
  mt = first + in % rows;
  nt = in / rows;
}

// XG: X' rows (X_F16: an fp16 matrix) or the conv3 gather (X_CONV3: input voxels [vox][Ci], padding taps read Z)
template <int WE, int XG, int TBM, int TBN, int NWV, int WGM>
__global__ __launch_bounds__((64 * NWV))
__attribute__((amdgpu_waves_per_eu((DT<WE, TBM, TBN, NWV, WGM>::OCC), (DT<WE, TBM, TBN, NWV, WGM>::OCC)))) void k_gemm_dma(Params p) {
  using T = DT<WE, TBM, TBN, NWV, WGM>;
  constexpr int S = T::S, BI = T::BI, BJ = T::BJ, NW = T::NW;
  constexpr int WTM = T::WTM, WTN = T::WTN;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[T::SMEM];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  uint32_t mt, nt;
  tile_order(p, blockIdx.x, mt, nt);
  const uint32_t mB = mt * TBM, nB = p.nbase + nt * TBN;
  const uint32_t nk = p.K / DBK;

  // ---- per-lane DMA sources (step 0) and per-step advances; instruction t of this wave is number 4 t + wave of
  //      the stage's list (NWV t + wave)
  uint32_t src[NW];                                   // byte offsets from X' / the weights (both < 4 GiB)
  uint32_t cv_it[XG == X_CONV3 ? T::WA : 1], cv_yx[XG == X_CONV3 ? T::WA : 1];   // conv3 row contexts
  uint32_t dst[NW];                                   // byte offset inside a stage
#pragma unroll
  for (int t = 0; t < NW; t++) {
    const int q = NWV * t + wave;
    if (t < T::WA) {                                  // X' rows 8q .. 8q+7
      const uint32_t r = 8 * q + lane / 8, c = (lane & 7) ^ ((r >> 1) & 7);
      uint32_t m = mB + r;
      m = m < p.M ? m : p.M - 1u;
      if constexpr (XG == X_CONV3) {
        // (oy | ox << 16) and the input frame of each of the three time taps (10 bits each)
        const RowCtx rc = row_ctx<X_CONV3>(p, m);
        uint32_t itp = 0;
#pragma unroll
        for (int kt3 = 0; kt3 < 3; kt3++) {
          int itg = rc.a + (int)p.padT + kt3 - 1;
          itg = itg < 0 ? 0 : (itg > (int)p.stride - 1 ? (int)p.stride - 1 : itg);
          const uint32_t it = p.ks > 1u ? (uint32_t)itg % p.ks : (uint32_t)itg - p.padL;
          itp |= it << (10 * kt3);
        }
        cv_it[t] = itp;
        cv_yx[t] = (uint32_t)rc.b | ((uint32_t)rc.c << 16);
        src[t] = 8 * c;
      } else {
        src[t] = (m * p.ldx + p.kx0 + 8 * c) * 2u;
      }
      dst[t] = q * 1024;
    } else if (T::WSPLIT ? t < T::WA + T::WC : q < T::NIA + T::NIC) {
      const int b = q - T::NIA;
      if constexpr (WE == W_F16) {                    // weight rows of ws columns 8b .. 8b+7
        const uint32_t r = 8 * b + lane / 8, c = (lane & 7) ^ ((r >> 1) & 7);
        src[t] = (wrow(p, nB + r) * p.wG + p.wk0 + 8 * c) * 2u;
      } else if constexpr (WE == W_Q4) {              // block b / 2, record b & 1: code row of column lane
        const uint32_t r = wrow(p, nB + 64 * (b >> 1) + lane);
        src[t] = ((r >> 6) * p.wG + (p.wk0 >> 5) + (b & 1)) * 1280u + (r & 63u) * 16u;
      } else {                                        // block b / 4, chunk b & 3
        const uint32_t r = wrow(p, nB + 64 * (b >> 2) + lane);
        src[t] = ((r >> 6) * p.wG + (p.wk0 >> 6)) * 4224u + (r & 63u) * 64u + (b & 3) * 16u;
      }
      dst[t] = T::A_BYTES + b * 1024;
    } else {
      const int b = q - (T::NIA + T::NIC);
      if constexpr (WE == W_Q4) {                     // (scale, min) word of block b / 2, record b & 1
        const uint32_t r = wrow(p, nB + 64 * (b >> 1) + lane);
        src[t] = ((r >> 6) * p.wG + (p.wk0 >> 5) + (b & 1)) * 1280u + 1024u + (r & 63u) * 4u;
      } else if constexpr (WE == W_Q8) {              // scale pair word of block b (repeats past the last block)
        const int bb = b < T::NBLK ? b : T::NBLK - 1;
        const uint32_t r = wrow(p, nB + 64 * bb + lane);
        src[t] = ((r >> 6) * p.wG + (p.wk0 >> 6)) * 4224u + 4096u + (r & 62u) * 2u;
      }
      dst[t] = T::A_BYTES + T::BC_BYTES + b * 256;
    }
  }
  constexpr uint32_t WSTEP = WE == W_F16 ? 128u : (WE == W_Q4 ? 2560u : 4224u);
  const uint32_t smem0 = lds_u32(smem);
  // issue part `part` (instructions part*NP ..) of step kt into stage st
  constexpr int NP = (NW + 2) / 3;
  auto issue = [&](uint32_t kt, int st, int part) __attribute__((always_inline)) {
    kt = kt < nk ? kt : nk - 1u;
    // conv3: the step's tap (uniform; Ci % 64 == 0, so a 64-k step stays inside one tap)
    uint32_t c0 = 0, kt3 = 0, ky = 0, kx = 0;
    if constexpr (XG == X_CONV3) {
      const uint32_t kg = kt * DBK, tap = kg / p.Ci, r9 = tap % 9u;
      c0 = kg - tap * p.Ci;
      kt3 = tap / 9u;
      ky = r9 / 3u;
      kx = r9 - 3u * ky;
    }
#pragma unroll
    for (int t = part * NP; t < (part + 1) * NP && t < NW; t++) {
      const uint32_t m0 = __builtin_amdgcn_readfirstlane(smem0 + st * T::STAGE + dst[t]);
      if (XG == X_CONV3 && t < T::WA) {
        const uint32_t it = (cv_it[t] >> (10 * kt3)) & 1023u;
        const int iy = (int)(cv_yx[t] & 0xffffu) + (int)ky - 1, ix = (int)(cv_yx[t] >> 16) + (int)kx - 1;
        const bool in = (uint32_t)iy < p.Hi && (uint32_t)ix < p.Wi;
        const size_t vox = ((size_t)it * p.Hi + (uint32_t)iy) * p.Wi + (uint32_t)ix;
        dma16a(in ? p.X + (vox * p.Ci + c0) * 2 + src[t] * 2 : p.Z, m0);
      } else if (t < T::WA) dma16(p.X + (size_t)kt * 128u, src[t], m0);
      else if (T::WSPLIT ? t < T::WA + T::WC : NWV * t + wave < T::NIA + T::NIC) dma16(p.W + (size_t)kt * WSTEP, src[t], m0);
      else dma4(p.W + (size_t)kt * WSTEP, src[t], m0);
    }
  };

  // ---- fragments
  const int wm = wave / T::WGN, wn = wave % T::WGN, l32 = lane & 31, hh = lane >> 5, sw = (l32 >> 1) & 7;
  const int rdA = (wm * WTM + l32) * 128;              // byte offset of the lane's first A row in a stage
  f32x16 acc[BI][BJ];
#pragma unroll
  for (int i = 0; i < BI; i++)
#pragma unroll
    for (int j = 0; j < BJ; j++) acc[i][j] = (f32x16){};
  f16x8 FA[2][BI], FB[2][BJ];
  // weight words of the current step: q4 code row (4 words = 4 sub-steps) + (scale, min); q8 two chunks + scale word
  u32x4 bc[BJ][WE == W_Q8 ? 2 : 1];
  uint32_t bs[BJ];
  uint32_t rodd = 0;                                   // q8: bit j = the column's weight row is odd (scale high half)
  if constexpr (WE == W_Q8) {
#pragma unroll
    for (int j = 0; j < BJ; j++) rodd |= (wrow(p, nB + wn * WTN + 32 * j + l32) & 1u) << j;
  }
  auto rdA_frag = [&](f16x8 *F, int st, int sub) __attribute__((always_inline)) {
    const uint8_t *sp = smem + st * T::STAGE + rdA + (((4 * hh + sub) ^ sw) & 7) * 16;
#pragma unroll
    for (int i = 0; i < BI; i++) F[i] = *(const f16x8 *)(sp + i * 32 * 128);
  };
  auto rdB_f16 = [&](f16x8 *F, int st, int sub) __attribute__((always_inline)) {
    const uint8_t *sp = smem + st * T::STAGE + T::A_BYTES + (wn * WTN + l32) * 128 + (((4 * hh + sub) ^ sw) & 7) * 16;
#pragma unroll
    for (int j = 0; j < BJ; j++) F[j] = *(const f16x8 *)(sp + j * 32 * 128);
  };
  auto rdB_codes = [&](int st) __attribute__((always_inline)) {
    const uint8_t *sb = smem + st * T::STAGE + T::A_BYTES;
#pragma unroll
    for (int j = 0; j < BJ; j++) {
      const int col = wn * WTN + 32 * j + l32, blk = col >> 6, cb = col & 63;
      if constexpr (WE == W_Q4) {
        bc[j][0] = *(const u32x4 *)(sb + (blk * 2 + hh) * 1024 + cb * 16);
        bs[j] = *(const uint32_t *)(sb + T::BC_BYTES + (blk * 2 + hh) * 256 + cb * 4);
      } else if constexpr (WE == W_Q8) {
        bc[j][0] = *(const u32x4 *)(sb + (blk * 4 + 2 * hh) * 1024 + cb * 16);
        bc[j][1] = *(const u32x4 *)(sb + (blk * 4 + 2 * hh + 1) * 1024 + cb * 16);
        bs[j] = *(const uint32_t *)(sb + T::BC_BYTES + blk * 256 + cb * 4);
      }
    }
  };
  // decode the weight fragments of sub-step `sub` from bc / bs. q4 takes the fast decode for every word here; a step
  // whose (scale, min) words are not all fast-path words is redone by fix_q4 after the sub-step's interleaved region,
  // so the common path stays one straight-line block.
  bool allfast = true;
  uint32_t fmask = 0;                                  // q4: bit j = word j of this step takes the fast decode
  f16x2 qs2[BJ], qm2[BJ];                              // q4: (s, s / 16) and (mn, mn) of the step's words
  uint32_t msk = 0x00F0000Fu, mag = 0x64006400u;
  asm volatile("" : "+v"(msk), "+v"(mag));
  auto decode = [&](f16x8 *F, int sub) __attribute__((always_inline)) {
    if constexpr (WE == W_Q4) {
#pragma unroll
      for (int j = 0; j < BJ; j++) F[j] = dq4_fast(bc[j][0][sub], qs2[j], qm2[j], msk, mag);
    } else if constexpr (WE == W_Q8) {
#pragma unroll
      for (int j = 0; j < BJ; j++) {
        const uint32_t sh = ((rodd >> j) & 1u) ? (bs[j] >> 16) : (bs[j] & 0xffffu);
        const f16x2 s2 = as_h2(sh | (sh << 16));
        const u32x4 &c = bc[j][sub >> 1];
        F[j] = (sub & 1) ? dq8(c.z, c.w, s2) : dq8(c.x, c.y, s2);
      }
    }
  };
  // chk: std::true_type where the tile holds words off the fast path (tile_q4_fast), std::false_type elsewhere
  auto fix_q4 = [&](f16x8 *F, int sub, auto chk) __attribute__((always_inline)) {
    if constexpr (WE == W_Q4 && decltype(chk)::value) {
      if (!allfast) {
#pragma unroll
        for (int j = 0; j < BJ; j++)
          if (!((fmask >> j) & 1u)) F[j] = dq4_slow(bc[j][0][sub], bs[j]);
      }
    }
  };
  auto check_q4 = [&](auto chk) __attribute__((always_inline)) {
    if constexpr (WE == W_Q4 && decltype(chk)::value) {
      fmask = 0;
#pragma unroll
      for (int j = 0; j < BJ; j++) fmask |= (uint32_t)q4n_fast_ok(bs[j]) << j;
      allfast = __all(fmask == (1u << BJ) - 1u);
    }
  };
  auto scales_q4 = [&]() __attribute__((always_inline)) {
    if constexpr (WE == W_Q4) {
#pragma unroll
      for (int j = 0; j < BJ; j++) {
        const f16x2 sm2 = as_h2(bs[j]);
        qs2[j] = (f16x2){sm2.x, sm2.x * (f16)0.0625f};
        qm2[j] = (f16x2){sm2.y, sm2.y};
      }
    }
  };
  auto mfma = [&](const f16x8 *A, const f16x8 *B) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < BJ; j++)
#pragma unroll
      for (int i = 0; i < BI; i++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[i], B[j], acc[i][j], 0, 0, 0);
  };
  // interleave a sub-step: MFMA, then a share of the VALU decode, then an LDS read
  auto sched = [&]() __attribute__((always_inline)) {
    constexpr int NMF = BI * BJ, NRD = BI + (WE == W_F16 ? BJ : 0);
    constexpr int NV = WE == W_F16 ? 0 : (WE == W_Q4 ? 18 * BJ : 16 * BJ);
    constexpr int VPM = (NV + NMF - 1) / NMF;
#pragma unroll
    for (int q = 0; q < NMF; q++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (VPM) __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
      if (q < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
  };

  // ---- prologue: stages 0 .. S-2 in full; the refill of stage S-1 goes out during step 0
#pragma unroll
  for (int s = 0; s < S - 1; s++)
#pragma unroll
    for (int part = 0; part < 3; part++) issue(s, s, part);
  // q4: when every (scale, min) word the tile reads takes the fast decode (ordinary weights), the K loop runs without
  // the per-step check and the fix-up branch of each sub-step, one straight-line block per sub-step
  bool tile_fast = true;
  if constexpr (WE == W_Q4) {
    // thread t reads column t % TBN in groups t / TBN, + NT / TBN, ...; 16 loads in flight per thread
    constexpr uint32_t GS = T::NT / TBN;
    const uint32_t ng = p.K >> 5, col = tid % TBN, r = wrow(p, nB + col);
    const uint8_t *wp = p.W + (size_t)((r >> 6) * p.wG + (p.wk0 >> 5) + tid / TBN) * 1280u + 1024u + (r & 63u) * 4u;
    bool ok = true;
    uint32_t g = tid / TBN;
    for (; g + 15 * GS < ng; g += 16 * GS, wp += 16 * GS * 1280u) {
      uint32_t w[16];
#pragma unroll
      for (int u = 0; u < 16; u++) w[u] = *(const uint32_t *)(wp + u * GS * 1280u);
#pragma unroll
      for (int u = 0; u < 16; u++) ok = ok & q4n_fast_ok(w[u]);
    }
    for (; g < ng; g += GS, wp += GS * 1280u) ok = ok & q4n_fast_ok(*(const uint32_t *)wp);
    tile_fast = __syncthreads_and(ok) != 0;
  }
  auto run = [&](auto chk) __attribute__((always_inline)) {
    wait_vm<(S - 2) * NW>();
    stage_barrier();
    rdA_frag(FA[0], 0, 0);
    if constexpr (WE == W_F16) {
      rdB_f16(FB[0], 0, 0);
    } else {
      rdB_codes(0);
      check_q4(chk);
      scales_q4();
      decode(FB[0], 0);
      fix_q4(FB[0], 0, chk);
    }
    int st = 0, pst = S - 1;
    uint32_t pk = S - 1;
    for (uint32_t kt = 0; kt < nk; kt++) {
#pragma unroll
      for (int sub = 0; sub < 3; sub++) {
        f16x8 *An = FA[(sub + 1) & 1], *Bn = FB[(sub + 1) & 1];
        rdA_frag(An, st, sub + 1);
        if constexpr (WE == W_F16) rdB_f16(Bn, st, sub + 1);
        issue(pk, pst, sub);
        if constexpr (WE != W_F16) decode(Bn, sub + 1);
        mfma(FA[sub & 1], FB[sub & 1]);
        sched();
        __builtin_amdgcn_sched_barrier(0);
        fix_q4(Bn, sub + 1, chk);
      }
      // the next stage has landed (own loads: only the refills of later stages may stay in flight), every wave is done
      // with this one (its fragments are in registers), then refill it with step kt + S
      const int sn = st + 1 == S ? 0 : st + 1;
      wait_vm<(S - 2) * NW>();
      wait_lgkm0();
      stage_barrier();
      pk = kt + S;
      pst = st;
      rdA_frag(FA[0], sn, 0);
      if constexpr (WE == W_F16) {
        rdB_f16(FB[0], sn, 0);
        mfma(FA[1], FB[1]);
      } else {
        // the last sub-step's weight fragments are decoded: the codes of the next step may replace them
        rdB_codes(sn);
        scales_q4();
        mfma(FA[1], FB[1]);
        decode(FB[0], 0);
      }
      sched();
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (WE == W_Q4) {
        check_q4(chk);
        fix_q4(FB[0], 0, chk);
      }
      st = sn;
    }
  };
  if (tile_fast) run(std::false_type{});
  else run(std::true_type{});
  wait_vm<0>();
  wait_lgkm0();
  stage_barrier();

  // ---- accumulators -> LDS, CR x CW at a time (32x32 layout: lane l, register r -> row 8 (r / 4) + 4 (l / 32) + r % 4,
  //      column l % 32), then the epilogue on each 128-column part of it (no barrier between the parts: they only read)
  float *sC = (float *)smem;
  constexpr int CLD = T::CLD;
#pragma unroll
  for (int v = 0; v < TBM / T::CR; v++)
#pragma unroll
    for (int h = 0; h < TBN / T::CW; h++) {
      // the wave's 32 x 32 blocks that lie in this part (a 1 x 4 layout's wave spans both row halves)
      const int r0 = wm * WTM - v * T::CR, c0 = wn * WTN - h * T::CW;
#pragma unroll
      for (int i = 0; i < BI; i++)
#pragma unroll
        for (int j = 0; j < BJ; j++) {
          const int br = r0 + i * 32, bc2 = c0 + j * 32;
          if (br >= 0 && br < T::CR && bc2 >= 0 && bc2 < T::CW) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
              const int row = br + 8 * (r >> 2) + 4 * hh + (r & 3);
              sC[row * CLD + bc2 + l32] = acc[i][j][r];
            }
          }
        }
      __syncthreads();
#pragma unroll
      for (int q = 0; q < T::CW / 128; q++)
        epilogue<T::NT>(p, sC + q * 128, CLD, T::CR, mB + v * T::CR, nB + h * T::CW + q * 128, tid);
      if (v + 1 < TBM / T::CR || h + 1 < TBN / T::CW) __syncthreads();
    }
}

template <int WE, int XG, int TBM, int TBN, int NWV = 4, int WGM = 2>
hipError_t launch_dma_one(const Params &p, hipStream_t s) {
  Params q = p;
  q.tilesM = (p.M + TBM - 1) / TBM;
  q.tilesN = (p.N - p.nbase + TBN - 1) / TBN;
  hipLaunchKernelGGL((k_gemm_dma<WE, XG, TBM, TBN, NWV, WGM>), dim3(q.tilesM * q.tilesN), dim3(64 * NWV), 0, s, q);
  return hipGetLastError();
}

template <int WE, int XG>
hipError_t launch_dma_we(const Params &p, unsigned bm, unsigned bn, unsigned cus, hipStream_t s) {
  if (bm == 256 && bn == 256) return launch_dma_one<WE, XG, 256, 256, 8>(p, s);
  if (bm == 256 && bn == 128) {
    // 8 waves (2 x 4, 128 x 32 each), one workgroup per CU; q4, whose 4-wave form fits two workgroups per CU, keeps
    // that when the grid holds more than one tile per CU (the same dma_wgs the planner scored the tile with)
    if constexpr (WE == W_Q4) {
      const uint64_t tiles = (uint64_t)((p.M + 255) / 256) * ((p.N - p.nbase + 127) / 128);
      if (dma_wgs(WE, 256, 128, tiles, cus) > 1) return launch_dma_one<WE, XG, 256, 128, 4>(p, s);
    }
    // f16 weights need no decode, so their 8 waves lay out 4 x 2 (64 x 64 each): 4 LDS fragments per 4 MFMAs
    // instead of 5 with 2 x 4 (128 x 32 each); conv3 13 x 92 x 160: 214 -> 207.5 us
    if constexpr (WE == W_F16) return launch_dma_one<WE, XG, 256, 128, 8, 4>(p, s);
    return launch_dma_one<WE, XG, 256, 128, 8>(p, s);
  }
  if (bm == 128 && bn == 256) return launch_dma_one<WE, XG, 128, 256>(p, s);
  if (bm == 128 && bn == 128) {
    // q4 with at most one tile per CU: 8 waves (2 x 4, 64 x 32 each, two per SIMD) instead of 4 at one per SIMD
    if constexpr (WE == W_Q4) {
      const uint64_t tiles = (uint64_t)((p.M + 127) / 128) * ((p.N - p.nbase + 127) / 128);
      if (dma_wgs(WE, 128, 128, tiles, cus) == 1) return launch_dma_one<WE, XG, 128, 128, 8>(p, s);
    }
    return launch_dma_one<WE, XG, 128, 128>(p, s);
  }
  return hipErrorInvalidValue;
}

// conv3 PixelNorm + SiLU, materialised once per input element (the fused prologue's exact fp16 values, xload8)
__global__ __launch_bounds__(256) void k_pnprep(Params p, uint16_t *xp) {
  const uint32_t c8 = p.Ci / 8;
  const uint64_t n = (uint64_t)p.nvox * c8;
  for (uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x; t < n; t += (uint64_t)gridDim.x * 256) {
    const uint64_t vox = t / c8;
    const uint32_t c0 = (uint32_t)(t - vox * c8) * 8;
    u32x4 v = *(const u32x4 *)(p.X + (vox * p.Ci + c0) * 2);
    const float sc = p.ST[vox];
    const f16x2 a = as_h2(v.x), b = as_h2(v.y), c = as_h2(v.z), d = as_h2(v.w);
    v = (u32x4){pack2(silu((float)a.x * sc), silu((float)a.y * sc)), pack2(silu((float)b.x * sc), silu((float)b.y * sc)),
                pack2(silu((float)c.x * sc), silu((float)c.y * sc)), pack2(silu((float)d.x * sc), silu((float)d.y * sc))};
    *(u32x4 *)(xp + vox * p.Ci + c0) = v;
  }
}

// X' of the rms / lnmod prologues, materialised once: Xp[m][k] = xload8 (the fused prologue's exact values); one
// workgroup per row, 8 k per thread and step
template <int XM>
__global__ __launch_bounds__(256) void k_xprep(Params p, uint16_t *xp) {
  const uint32_t k8 = p.K / 8, m = blockIdx.x;
  uint16_t *dst = xp + (size_t)m * p.K;
#pragma unroll 2
  for (uint32_t kq = threadIdx.x; kq < k8; kq += 256) *(u32x4 *)(dst + 8 * kq) = xload8<XM, 1>(p, m, RowCtx{0, 0, 0}, 8 * kq);
}

}  // namespace

bool gemm_dma_ok(const Params &p, int we, int xm, uint64_t wbytes) {
  if (xm != X_F16 && xm != X_RMS && xm != X_LNMOD && xm != X_CONV3) return false;
  if (xm == X_CONV3) {
    // 64-k steps inside one tap; input frames of the three time taps packed in 10 bits; (oy, ox) in 16
    if (p.Ci % 64 != 0 || p.stride > 1024 || p.ks > 1024 || p.Ho > 65535 || p.Wo > 65535 || p.nvox == 0xffffffffu)
      return false;
  } else {
    // 32-bit lane offsets from the X' base
    const uint64_t xbytes = xm == X_F16 ? ((uint64_t)p.M * p.ldx + p.kx0 + p.K) * 2 : (uint64_t)p.M * p.K * 2;
    if (xbytes >= (1ull << 32)) return false;
  }
  if (wbytes >= (1ull << 32)) return false;
  if (p.K % DBK != 0 || p.K == 0) return false;
  if (xm == X_F16 && !(p.flags & F_XALIGN8)) return false;
  if (we == W_F16 && !(p.flags & F_WALIGN8)) return false;
  if (we == W_Q4 && p.wk0 % 32 != 0) return false;
  if (we == W_Q8 && p.wk0 % 64 != 0) return false;
  return we == W_F16 || we == W_Q4 || we == W_Q8;
}

hipError_t launch_xprep(const Params &p, int xm, uint16_t *xp, hipStream_t s) {
  if (xm == X_CONV3) {
    const uint64_t n = (uint64_t)p.nvox * (p.Ci / 8);
    const unsigned blocks = (unsigned)(n / 256 < 4096 ? (n + 255) / 256 : 4096);
    if (n) hipLaunchKernelGGL(k_pnprep, dim3(blocks), dim3(256), 0, s, p, xp);
    return hipGetLastError();
  }
  if (p.M == 0) return hipSuccess;
  if (xm == X_RMS) hipLaunchKernelGGL(k_xprep<X_RMS>, dim3(p.M), dim3(256), 0, s, p, xp);
  else if (xm == X_LNMOD) hipLaunchKernelGGL(k_xprep<X_LNMOD>, dim3(p.M), dim3(256), 0, s, p, xp);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

// The tile: each candidate scored by its relative per-CU rate times the fraction of workgroup slots (one or two per
// CU, as the tile's LDS allows) that hold real work over the rounds the grid needs.
// workgroups per CU of a tile for a grid of `tiles` (q4 256 x 128: 8 waves when the grid has one tile per CU at most)
unsigned dma_wgs(int we, unsigned m, unsigned n, uint64_t tiles, unsigned cus) {
  if (m == 256 && n == 256) return 1;
  if (m == 256 && (we != W_Q4 || tiles <= cus)) return 1;           // 8 waves
  if (m == 128 && n == 128 && we == W_Q4 && tiles <= cus) return 1;   // 8 waves
  if (we == W_F16) return m == 128 && n == 128 ? (DT<W_F16, 128, 128>::WGS) : (DT<W_F16, 128, 256>::WGS);
  if (we == W_Q4) return m == 128 && n == 128 ? DT<W_Q4, 128, 128>::WGS : (m == 128 ? DT<W_Q4, 128, 256>::WGS : DT<W_Q4, 256, 128>::WGS);
  return m == 128 && n == 128 ? DT<W_Q8, 128, 128>::WGS : (m == 128 ? DT<W_Q8, 128, 256>::WGS : DT<W_Q8, 256, 128>::WGS);
}

void dma_tile(uint32_t M, uint32_t N, int we, int xg, unsigned cus, unsigned *bm, unsigned *bn) {
  auto per_cu = [&](unsigned m, unsigned n) -> unsigned {
    return dma_wgs(we, m, n, (uint64_t)((M + m - 1) / m) * ((N + n - 1) / n), cus);
  };
  // relative per-CU rates measured on MI355X at 4096^3 (f16 prologue), per weight encoding: 256 x 256 and (f16, q8)
  // 256 x 128 run 8 waves (two per SIMD), the others 4; the quantised weights favour 256-row tiles (each decoded
  // weight feeds four 32-row blocks instead of two)
  struct C { unsigned m, n; double rate; };
  const C c16[] = {{256, 256, 1.0}, {128, 256, 0.94}, {256, 128, 0.99}, {128, 128, 0.91}};
  const C cq4[] = {{256, 256, 1.0}, {128, 256, 0.68}, {256, 128, 0.91}, {128, 128, 0.68}};
  const C cq8[] = {{256, 256, 1.0}, {128, 256, 0.75}, {256, 128, 0.84}, {128, 128, 0.78}};
  // the conv3 gather computes each row's tap address per step (f16 weights, 13 x 92 x 160 x 128 clip: 256 x 128 with
  // 8 waves 244 us, 128 x 128 (two workgroups per CU) 257, 256 x 256 382 and 128 x 256 409 with 4 waves)
  const C cg[] = {{256, 256, 0.66}, {128, 256, 0.62}, {256, 128, 1.05}, {128, 128, 1.0}};
  const C *cand = xg == X_CONV3 ? cg : (we == W_F16 ? c16 : (we == W_Q4 ? cq4 : cq8));
  double best = -1.0;
  for (int ci = 0; ci < 4; ci++) {
    const C &c = cand[ci];
    if (c.n == 256 && N <= 128) continue;
    if (c.m == 256 && M <= 128) continue;
    const uint64_t tiles = (uint64_t)((M + c.m - 1) / c.m) * ((N + c.n - 1) / c.n), slots = (uint64_t)cus * per_cu(c.m, c.n);
    const double rounds = (double)((tiles + slots - 1) / slots);
    const double useful = (double)M * N / ((double)c.m * c.n * rounds * slots);
    // q4 256 x 128 with 8 waves (a grid of one tile per CU at most): 2048 x 4096 x 4096 in 87.7 us against 143.7 for
    // twice the work at 256 x 256
    double rate = (we == W_Q4 && c.m == 256 && c.n == 128 && tiles <= cus) ? 0.80 : c.rate;
    // q4 128 x 128 with 8 waves (at most one tile per CU): DiT QKV's last 1024 columns as 256 such tiles instead of
    // 128 of 256 x 128 on half the CUs, 272 -> 265 us per call
    if (we == W_Q4 && c.m == 128 && c.n == 128 && tiles <= cus) rate = 0.6;
    const double score = rate * useful;
    if (score > best + 1e-9) { best = score; *bm = c.m; *bn = c.n; }
  }
}

static hipError_t launch_dma_x(const Params &p, int we, unsigned bm, unsigned bn, unsigned cus, hipStream_t s) {
  switch (we) {
  case W_Q4: return launch_dma_we<W_Q4, X_F16>(p, bm, bn, cus, s);
  case W_Q8: return launch_dma_we<W_Q8, X_F16>(p, bm, bn, cus, s);
  case W_F16: return launch_dma_we<W_F16, X_F16>(p, bm, bn, cus, s);
  }
  return hipErrorInvalidValue;
}

// Tail columns: when the grid's last round of tiles would leave at least half of the workgroup slots empty, the
// whole rounds run as one launch over the first columns (as many whole column bands of tiles as they hold) and the
// remaining columns as a second launch with the tile dma_tile picks for them (smaller tiles, more of them). Every tile
// sums K in the same order, so the output is the same bits as one launch. DiT QKV (576 tiles of 256 x 256 on 256 CUs,
// 2.25 rounds): 512 tiles, then the last 1024 columns in 128 x 128 tiles. P0K_DMA_TAIL=0 keeps one launch.
void dma_tail(uint32_t M, uint32_t N, int we, unsigned bm, unsigned bn, unsigned cus, uint32_t *ncut, unsigned *bm2,
              unsigned *bn2) {
  *ncut = N;
  *bm2 = bm;
  *bn2 = bn;
  const uint32_t tilesM = (M + bm - 1) / bm, tilesN = (N + bn - 1) / bn, T = tilesM * tilesN;
  const uint32_t slots = cus * dma_wgs(we, bm, bn, T, cus), full = T / slots * slots, tail = T - full;
  if (tail == 0 || 2 * tail > slots || full < tilesM) return;
  const uint32_t nA = full / tilesM;                           // column bands of the first launch
  if (nA >= tilesN) return;
  *ncut = nA * bn;
  dma_tile(M, N - *ncut, we, X_F16, cus, bm2, bn2);
}

hipError_t launch_gemm_dma(const Params &p, int we, int xg, unsigned bm, unsigned bn, unsigned cus, bool tail,
                           hipStream_t s) {
  if (xg != X_CONV3) {
    uint32_t ncut = p.N;
    unsigned bm2 = bm, bn2 = bn;
    if (tail) dma_tail(p.M, p.N, we, bm, bn, cus, &ncut, &bm2, &bn2);
    if (ncut >= p.N) return launch_dma_x(p, we, bm, bn, cus, s);
    Params a = p, b = p;
    a.N = ncut;                                                 // epilogue bounds: the first launch's columns only
    a.nbase = 0;
    b.nbase = ncut;
    hipError_t e = launch_dma_x(a, we, bm, bn, cus, s);
    if (e != hipSuccess) return e;
    return launch_dma_x(b, we, bm2, bn2, cus, s);
  }
  if (xg == X_CONV3) {
    switch (we) {
    case W_Q4: return launch_dma_we<W_Q4, X_CONV3>(p, bm, bn, cus, s);
    case W_Q8: return launch_dma_we<W_Q8, X_CONV3>(p, bm, bn, cus, s);
    case W_F16: return launch_dma_we<W_F16, X_CONV3>(p, bm, bn, cus, s);
    }
    return hipErrorInvalidValue;
  }
  return hipErrorInvalidValue;
}

}  // namespace p0k
