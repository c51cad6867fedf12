// p0k_attention.hip — flash attention over the `heads` output of the QKV gemm (src/ops/attention.js:168-201), head
// size 128, on gfx950 matrix cores.
//
//   Q [Hq][Lq][128] f16, K / V [Hkv][Lk][128] f16 (head-major, as the heads epilogue writes them), O [Lq][ldo] f16
//   token-major at column h*128. Query head h reads kv head h / (Hq / Hkv). mode 0: no mask; 1: key j visible to query
//   i iff j <= min(i, nvalid - 1); 2: j < nvalid. Scores s = scale * q.k (scale defaults to 1/sqrt(128)), optionally
//   soft-capped to cap * tanh(s / cap); O = softmax(s) V with an exact online softmax in fp32.
//
// One workgroup (4 waves) owns 128 queries of one head; each wave owns 32 of them and keeps its Q rows in registers.
// Everything is computed transposed, so that a lane owns ONE query and the softmax statistics stay in the lane:
//   S^T (keys x queries) = K Q^T           v_mfma_f32_32x32x16_f16, A = K from LDS, B = Q^T from registers
//   O^T (d x queries)   += V^T P           A = V^T from LDS, B = P = exp(S - m) from the S^T registers (fp16)
// In the 32x32 layout lane l holds column l % 32 (its query) and 16 rows 8 (r/4) + 4 (l/32) + r%4, so a row maximum
// or sum is a reduction over the lane's registers plus one exchange with lane l ^ 32. The 16 keys a lane contributes
// to one P.V step are exactly the keys its S^T registers hold, so P never leaves the registers; V is staged in LDS
// transposed ([d][key]) so those keys are two 8-byte reads. Keys come in tiles of 64 through double-buffered LDS (the
// next tile's global loads are issued before this tile's MFMAs); both LDS tiles are XOR-swizzled so the 16-byte K reads
// and the 8-byte V reads of a wave hit distinct banks (the V swizzle also folds in d >> 5, so the rows d and d + 32 that
// one read instruction pairs land in different banks). K arrives by the load-to-LDS path; V is transposed through
// registers. Two waves per SIMD (256 registers each) let one wave's softmax run under the other's MFMAs.
#include "p0k_device.h"
#include "p0k_launch.h"

namespace p0k {

#ifndef P0K_AT_BQ
#define P0K_AT_BQ 128
#endif
constexpr int AT_BQ = P0K_AT_BQ, AT_BK = 64, AT_NT = 2 * AT_BQ, AT_NW = AT_NT / 64;   // 32 queries per wave

template <bool CAP>
__global__ __launch_bounds__(AT_NT, 2 * 256 / AT_NT) void k_attention(AttnParams p) {
  __shared__ __attribute__((aligned(16))) f16 sK[2][AT_BK * 128];   // [key][d], 16-byte chunk c at c ^ (key & 15)
  __shared__ __attribute__((aligned(16))) f16 sV[2][128 * AT_BK];   // [d][key], 4-key unit u at u ^ (((d >> 1) ^ (d >> 5)) & 15)

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
  // V staging: thread (vkg, vdc, vh) holds keys 4 vkg + VPT vh .. + VPT-1 of d 8 vdc .. + 7
  constexpr int VPT = 4 * 256 / AT_NT;                   // keys per thread
  u32x4 vr[VPT];
  const uint32_t vkg = tid & 15, vdc = (tid >> 4) & 15, vh = tid >> 8;
  // K goes global -> LDS by the load-to-LDS path: instruction i of wave w fills keys 4 (4 i + w) .. + 3 (1 KB), lane l
  // the 16-byte slot l % 16 of key l / 16, i.e. logical chunk (l % 16) ^ (key & 15)
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
  auto gload = [&](uint32_t t) {
    const uint32_t k0 = t * AT_BK;
#pragma unroll
    for (int i = 0; i < VPT; i++) {
      const uint32_t vk = k0 + 4 * vkg + VPT * vh + i;
      vr[i] = *(const u32x4 *)(Vb + (size_t)(vk < p.Lk ? vk : p.Lk - 1u) * 128 + vdc * 8);
    }
  };
  auto lstore = [&](int b) {
    if constexpr (VPT == 4) {
      // The 16 threads of one d cover the 16 units of its row (half the banks), so the two d a 32-lane half writes
      // per instruction must differ in parity (row parity picks the bank half): odd 16-lane groups write the rows
      // of each pair (2w, 2w+1) in swapped order, picking the halves with a lane-dependent v_perm selector.
      const uint32_t odd = (tid >> 4) & 1u;
      const uint32_t s0 = odd ? 0x07060302u : 0x05040100u, s1 = odd ? 0x05040100u : 0x07060302u;
#pragma unroll
      for (int w = 0; w < 4; w++) {
        const uint32_t a0 = vr[0][w], a1 = vr[1][w], a2 = vr[2][w], a3 = vr[3][w];
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const uint32_t sel = h ? s1 : s0, d = vdc * 8 + 2 * w + (h ^ odd);
          *(u32x2 *)(sV[b] + d * AT_BK + ((vkg ^ (((d >> 1) ^ (d >> 5)) & 15u)) * 4)) = (u32x2){perm(a1, a0, sel), perm(a3, a2, sel)};
        }
      }
    } else {                                               // two keys per thread: half of a 4-key unit
      const uint16_t *v0 = (const uint16_t *)&vr[0], *v1 = (const uint16_t *)&vr[1];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const uint32_t d = vdc * 8 + j;
        *(uint32_t *)(sV[b] + d * AT_BK + ((vkg ^ (((d >> 1) ^ (d >> 5)) & 15u)) * 4) + 2 * vh) =
            (uint32_t)v0[j] | ((uint32_t)v1[j] << 16);
      }
    }
  };


  f32x16 oacc[4];
#pragma unroll
  for (int i = 0; i < 4; i++) oacc[i] = (f32x16){};
  float m = -1.0e30f, l = 0.0f;

  if (ntile) {
    kdma(0, 0);
    gload(0);
    lstore(0);
  }
  __builtin_amdgcn_s_waitcnt(0x0f70);                     // vmcnt(0): this wave's K rows have landed
  __syncthreads();
  for (uint32_t t = 0; t < ntile; t++) {
    const int b = t & 1;
    const uint32_t k0 = t * AT_BK;
    if (t + 1 < ntile) {
      gload(t + 1);
      kdma(t + 1, b ^ 1);                                   // the other K buffer: every wave left it at the last barrier
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
        for (int r = 0; r < 16; r++) sacc[kb][r] = p.cap * tanhf(sacc[kb][r] * p.scale / p.cap);
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
    const float mn = fmaxf(m, mxl);
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
    if (__any(mn != m)) {                                       // rescale only when some row's maximum moved
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
      const uint32_t u1 = 8 * kb + 4 * h2 + gh, u2 = u1 + 2;   // 4-key units of the lane's 8 keys
#pragma unroll
      for (int db = 0; db < 4; db++) {
        const uint32_t d = 32 * db + l32, sw = ((d >> 1) ^ (d >> 5)) & 15u;
        const u32x2 lo = *(const u32x2 *)(sV[b] + d * AT_BK + ((u1 ^ sw) * 4));
        const u32x2 hi = *(const u32x2 *)(sV[b] + d * AT_BK + ((u2 ^ sw) * 4));
        const f16x8 av = __builtin_bit_cast(f16x8, (u32x4){lo.x, lo.y, hi.x, hi.y});
        oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bp, oacc[db], 0, 0, 0);
      }
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
#pragma unroll
    for (int q = 0; q < 15; q++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
    __builtin_amdgcn_sched_barrier(0);
    if (t + 1 < ntile) lstore(b ^ 1);
    __builtin_amdgcn_s_waitcnt(0x0f70);                   // vmcnt(0): the next K tile has landed
    __syncthreads();
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

hipError_t launch_attention(const AttnParams &p, hipStream_t s) {
  if (p.Lq == 0 || p.Hq == 0) return hipSuccess;
  dim3 grid(((p.Lq + AT_BQ - 1) / AT_BQ) * p.Hq);
  if (p.cap > 0.0f) hipLaunchKernelGGL(k_attention<true>, grid, dim3(AT_NT), 0, s, p);
  else hipLaunchKernelGGL(k_attention<false>, grid, dim3(AT_NT), 0, s, p);
  return hipGetLastError();
}

}  // namespace p0k
