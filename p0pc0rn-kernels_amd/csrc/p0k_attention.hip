// p0k_attention.hip — flash attention over the `heads` output of the QKV gemm (src/ops/attention.js:168-201), head
// size 128, on gfx950 matrix cores.
//
//   Q [Hq][Lq][128] f16, K / V [Hkv][Lk][128] f16 (head-major, as the heads epilogue writes them), O [Lq][ldo] f16
//   token-major at column h*128. Query head h reads kv head h / (Hq / Hkv). mode 0: no mask; 1: key j visible to query
//   i iff j <= min(i, nvalid - 1); 2: j < nvalid. Scores s = scale * q.k (scale defaults to 1/sqrt(128)), optionally
//   soft-capped to cap * tanh(s / cap); O = softmax(s) V with an exact online softmax in fp32.
//
// One workgroup owns 128 queries of one head (4 waves, 32 queries each, two workgroups per CU; a 256-query, 8-wave
// variant is selectable for tuning); each wave keeps its Q rows in registers. Everything is computed transposed, so
// that a lane owns ONE query and the softmax statistics stay in it:
//   S^T (keys x queries) = K Q^T           v_mfma_f32_32x32x16_f16, A = K from LDS, B = Q^T from registers
//   O^T (d x queries)   += V^T P           A = V^T from LDS, B = P = exp(S - m) from the S^T registers (fp16)
// In the 32x32 layout lane l holds column l % 32 (its query) and 16 rows 8 (r/4) + 4 (l/32) + r%4, so a row maximum
// or sum is a reduction over the lane's registers plus one exchange with lane l ^ 32. The 16 keys a lane contributes
// to one P.V step are exactly the keys its S^T registers hold, so P never leaves the registers. Keys come in tiles of
// 64 through a two-stage LDS ring (the next tile's loads are issued before this tile's MFMAs); K and V both arrive
// by the load-to-LDS path in their HBM layout [key][d], and the V^T operand is read with the transposing
// ds_read_b64_tr_b16 (four keys of one d per lane). Both tiles are XOR-swizzled so the 16-byte K reads and the
// transposed V reads of a wave hit distinct banks. Two waves per SIMD (256 registers each) let one wave's softmax
// run under the other's MFMAs.
#include "p0k_device.h"
#include "p0k_launch.h"
#include <cstdlib>

namespace p0k {

#ifndef P0K_AT_S
#define P0K_AT_S 2
#endif
constexpr int AT_S = P0K_AT_S, AT_BK = 64;

// AT_BQ queries per workgroup (128 or 256), 32 per wave
template <int AT_BQ, bool CAP>
__global__ __launch_bounds__((2 * AT_BQ), (512 / (2 * AT_BQ))) void k_attention(AttnParams p) {
  constexpr int AT_NT = 2 * AT_BQ, AT_NW = AT_NT / 64;
  __shared__ __attribute__((aligned(16))) f16 sK[AT_S][AT_BK * 128];   // [key][d], 16-byte chunk c at c ^ (key & 15)
  __shared__ __attribute__((aligned(16))) f16 sV[AT_S][AT_BK * 128];   // [key][d], 16-byte chunk c at c ^ 4 (key & 3)

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, gh = lane >> 5, l32 = lane & 31;
  // Workgroups go round-robin to the 8 XCDs; regroup them so each XCD walks whole heads (all query blocks of a head
  // in a row): the head's K / V (Lk x 256 B) then stays in that XCD's L2 instead of being fetched once per query block
  const uint32_t nqb = (p.Lq + AT_BQ - 1) / AT_BQ, nblk = nqb * p.Hq, b0 = blockIdx.x;
  const uint32_t lin = (nblk & 7u) == 0u ? (b0 & 7u) * (nblk >> 3) + (b0 >> 3) : b0;
  const uint32_t h = lin / nqb, hk = h / (p.Hq / p.Hkv);
  const uint32_t q0 = (lin - h * nqb) * AT_BQ, qw = q0 + wave * 32 + l32;
  const uint32_t qc = qw < p.Lq ? qw : p.Lq - 1u;

  // this lane's query row: 8 steps of 16 d, lane half gh holds d = 16 s + 8 gh .. + 7
  f16x8 qf[8];
  const uint16_t *qrow = p.Q + ((size_t)h * p.Lq + qc) * 128;
#pragma unroll
  for (int s = 0; s < 8; s++) qf[s] = *(const f16x8 *)(qrow + 16 * s + 8 * gh);

  uint32_t kend = p.Lk;
  if (p.mode == 1) {
    const uint32_t last = q0 + AT_BQ - 1 < p.nvalid - 1 ? q0 + AT_BQ - 1 : p.nvalid - 1;
    kend = p.Lk < last + 1 ? p.Lk : last + 1;
  } else if (p.mode == 2) {
    kend = p.Lk < p.nvalid ? p.Lk : p.nvalid;
  }
  // the keys this lane's query may see
  uint32_t qlim = p.Lk;
  if (p.mode == 1) qlim = (qc < p.nvalid - 1 ? qc : p.nvalid - 1) + 1;
  else if (p.mode == 2) qlim = p.nvalid;
  qlim = qlim < p.Lk ? qlim : p.Lk;
  const uint32_t ntile = (kend + AT_BK - 1) / AT_BK;
  const float sl2 = p.scale * 1.4426950408889634f;

  const uint16_t *Kb = p.K + (size_t)hk * p.Lk * 128, *Vb = p.V + (size_t)hk * p.Lk * 128;
  // K and V go global -> LDS by the load-to-LDS path: instruction i of wave w fills keys 4 (NW i + w) .. + 3 (1 KB),
  // lane l the 16-byte slot l % 16 of key l / 16, i.e. logical chunk (l % 16) ^ (key & 15) of K, (l % 16) ^ 4 (key & 3)
  // of V
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t sk0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)&sK[0][0];
  auto kdma = [&](uint32_t t, int b) {
    const uint32_t k0 = t * AT_BK;
#pragma unroll
    for (int i = 0; i < 16 / AT_NW; i++) {
      const uint32_t kr = 4 * (AT_NW * i + wv) + lane / 16, key = k0 + kr, c = (lane & 15) ^ (kr & 15);
      const uint32_t off = ((key < p.Lk ? key : p.Lk - 1u) * 128 + c * 8) * 2;
      const uint32_t m0 = __builtin_amdgcn_readfirstlane(sk0 + (uint32_t)(b * AT_BK * 128 + 4 * (AT_NW * i + wv) * 128) * 2);
      asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(m0), "v"(off), "s"(Kb) : "memory");
    }
  };
  const uint32_t sv0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)&sV[0][0];
  auto vdma = [&](uint32_t t, int b) {
    const uint32_t k0 = t * AT_BK;
#pragma unroll
    for (int i = 0; i < 16 / AT_NW; i++) {
      const uint32_t kr = 4 * (AT_NW * i + wv) + lane / 16, key = k0 + kr, c = (lane & 15) ^ (4 * (kr & 3));
      const uint32_t off = ((key < p.Lk ? key : p.Lk - 1u) * 128 + c * 8) * 2;
      const uint32_t m0 = __builtin_amdgcn_readfirstlane(sv0 + (uint32_t)(b * AT_BK * 128 + 4 * (AT_NW * i + wv) * 128) * 2);
      asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(m0), "v"(off), "s"(Vb) : "memory");
    }
  };
  f32x16 oacc[4];
#pragma unroll
  for (int i = 0; i < 4; i++) oacc[i] = (f32x16){};
  float m = -1.0e30f, l = 0.0f;

  // AT_S-stage ring: tile t lives in buffer t % AT_S; tile t + AT_S - 1 is issued at the top of tile t into the buffer
  // every wave left at the barrier that ended tile t - 1. A wave's own loads complete in order, so waiting until at
  // most (AT_S - 2) tiles' worth of them are outstanding means its share of the next tile has landed.
  constexpr int PER = 32 / AT_NW;                           // load instructions per wave per tile (K and V)
  constexpr int NOUT = (AT_S - 2) * PER;
  constexpr int WAIT_RING = (NOUT & 15) | ((NOUT >> 4) << 14) | 0x0f70;
#pragma unroll
  for (int i = 0; i < AT_S - 1; i++)
    if ((uint32_t)i < ntile) {
      kdma(i, i);
      vdma(i, i);
    }
  if (ntile >= (uint32_t)(AT_S - 1)) __builtin_amdgcn_s_waitcnt(WAIT_RING);
  else __builtin_amdgcn_s_waitcnt(0x0f70);
  __syncthreads();
  int b = 0;
  for (uint32_t t = 0; t < ntile; t++) {
    const uint32_t k0 = t * AT_BK;
    if (t + AT_S - 1 < ntile) {
      const int bn = b == 0 ? AT_S - 1 : b - 1;
      kdma(t + AT_S - 1, bn);
      vdma(t + AT_S - 1, bn);
    }

    // ---- S^T for keys k0 .. k0+63: two 32-key blocks
    // (the two key blocks' MFMA chains alternate, and each K fragment read is issued one MFMA ahead of its use)
    f32x16 sacc[2];
    sacc[0] = (f32x16){};
    sacc[1] = (f32x16){};
#pragma unroll
    for (int s = 0; s < 8; s++)
#pragma unroll
      for (int kb = 0; kb < 2; kb++) {
        const uint32_t key = 32 * kb + l32;
        const f16x8 a = *(const f16x8 *)(sK[b] + key * 128 + (((2 * s + gh) ^ (key & 15u)) * 8));
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[s], sacc[kb], 0, 0, 0);
      }
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
    for (int q = 0; q < 14; q++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    __builtin_amdgcn_sched_barrier(0);
    // ---- scores to the log2 domain: max over the raw scores (the scale is positive), then exp2(s * sl2 - m) with one
    //      FMA per score. Soft cap: s -> cap * tanh(s * scale / cap) first. Keys past the lane's limit are masked only
    //      in tiles that reach past some lane's limit (a wave-uniform test).
    float sf = sl2;
    if constexpr (CAP) {
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int r = 0; r < 16; r++) sacc[kb][r] = p.cap * (2.0f * sigmoid(2.0f * sacc[kb][r] * p.scale / p.cap) - 1.0f);
      sf = 1.4426950408889634f;
    }
    const uint32_t kl = qlim > k0 ? qlim - k0 : 0u;           // keys of this tile the lane's query sees: [0, kl)
    if (__any(kl < (uint32_t)AT_BK)) {
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const uint32_t key = 32 * kb + 8 * (r >> 2) + 4 * gh + (r & 3);
          sacc[kb][r] = key < kl ? sacc[kb][r] : -1.0e30f;
        }
    }
    float mx = -1.0e30f;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int r = 0; r < 16; r++) mx = fmaxf(mx, sacc[kb][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    // m: running maximum in the log2 domain (-1e30: none yet)
    const float mxl = mx <= -1.0e29f ? -1.0e30f : mx * sf;
    // the maximum the exponents subtract stays where it is until some row's maximum grows past it by more than 8
    // (P <= 2^8 = 256 meanwhile: exact enough in fp16, and O and l keep the same common factor, which the final
    // division removes), so most tiles skip the rescale of O
    const float mn = __any(mxl > m + 8.0f) ? fmaxf(m, mxl) : m;
    // a masked score (-1e30) underflows exp2 to 0; a row with no visible key yet subtracts 0 instead of -1e30
    const float mns = mn <= -1.0e29f ? 0.0f : mn;
    float ps = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const float e = __builtin_amdgcn_exp2f(fmaf(sacc[kb][r], sf, -mns));
        sacc[kb][r] = e;
        ps += e;
      }
    if (__any(mn != m)) {                                       // rescale only when the subtracted maximum moved
      const float alpha = __builtin_amdgcn_exp2f(m - mn);
      l = l * alpha;
#pragma unroll
      for (int db = 0; db < 4; db++) oacc[db] *= alpha;
    }
    m = mn;
    l += ps;

    // ---- O^T += V^T P over four 16-key steps
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int kb = c >> 1, h2 = c & 1;
      const f16x8 bp = {(f16)sacc[kb][8 * h2 + 0], (f16)sacc[kb][8 * h2 + 1], (f16)sacc[kb][8 * h2 + 2],
                        (f16)sacc[kb][8 * h2 + 3], (f16)sacc[kb][8 * h2 + 4], (f16)sacc[kb][8 * h2 + 5],
                        (f16)sacc[kb][8 * h2 + 6], (f16)sacc[kb][8 * h2 + 7]};
#pragma unroll
      for (int db = 0; db < 4; db++) {
        // transposed read: lane 4 j + a of each 16-lane group addresses key j, d 4 a .. 4 a + 3; lane 4 a + b then
        // receives d 4 a + b of keys j = 0..3. Lanes 16..31 of a half take the next 16 d; half gh the keys 4 gh ..
        const uint32_t kr = 32 * kb + 16 * h2 + 4 * gh + ((lane >> 2) & 3), c = 4 * db + 2 * ((lane >> 4) & 1) + ((lane >> 1) & 1);
        const f16 *va = sV[b] + kr * 128 + ((c ^ (4 * (kr & 3))) * 8) + 4 * (lane & 1);
        typedef short v4s __attribute__((ext_vector_type(4)));
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s *)va);
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s *)(va + 8 * 128));
        const f16x8 av = __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bp, oacc[db], 0, 0, 0);
      }
    }
    // (this phase is left to the compiler's schedule: pinning each MFMA behind two transposed V reads, as the S phase
    // pins its K reads, ran 249-251 against 242-244 us)
    if (t + AT_S - 1 < ntile) __builtin_amdgcn_s_waitcnt(WAIT_RING);   // this wave's share of tile t + 1 has landed
    else __builtin_amdgcn_s_waitcnt(0x0f70);
    __syncthreads();
    b = b == AT_S - 1 ? 0 : b + 1;
  }

  // ---- O = O^T / l: lane writes its query's 128 values in runs of 4 d
  const float lt = l + __shfl_xor(l, 32, 64);
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
  if (qw < p.Lq) {
    uint16_t *orow = p.O + (size_t)qw * p.ldo + h * 128;
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
      for (int g4 = 0; g4 < 4; g4++) {
        const uint32_t d = 32 * db + 8 * g4 + 4 * gh;
        *(u32x2 *)(orow + d) = (u32x2){pack2(oacc[db][4 * g4] * inv, oacc[db][4 * g4 + 1] * inv),
                                       pack2(oacc[db][4 * g4 + 2] * inv, oacc[db][4 * g4 + 3] * inv)};
      }
  }
}

int attention_bq(uint32_t Lq, uint32_t Hq, int cus, int force) {
  if (force == 128 || force == 256) return force;                 // tuning / tests (P0K_ATTN_BQ)
  // 128 (two workgroups per CU). 256 queries per workgroup halve the LDS fill per query but run one workgroup per CU:
  // 24 heads x 4096 queries, 300 us vs 280 us (its 384 blocks leave half the CUs idle in the second round, where
  // the 768 blocks of 128 let the last third of a CU's blocks run alone and faster)
  (void)Lq;
  (void)Hq;
  (void)cus;
  return 128;
}

hipError_t launch_attention(const AttnParams &p, int cus, int force_bq, hipStream_t s) {
  if (p.Lq == 0 || p.Hq == 0) return hipSuccess;
  const int bq = attention_bq(p.Lq, p.Hq, cus, force_bq);
  dim3 grid(((p.Lq + bq - 1) / bq) * p.Hq);
  if (bq == 256) {
    if (p.cap > 0.0f) hipLaunchKernelGGL((k_attention<256, true>), grid, dim3(512), 0, s, p);
    else hipLaunchKernelGGL((k_attention<256, false>), grid, dim3(512), 0, s, p);
  } else {
    if (p.cap > 0.0f) hipLaunchKernelGGL((k_attention<128, true>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((k_attention<128, false>), grid, dim3(256), 0, s, p);
  }
  return hipGetLastError();
}

}  // namespace p0k
