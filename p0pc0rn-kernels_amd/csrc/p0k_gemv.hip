// p0k_gemv.hip — the decode path of `gemm` (M <= 16): memory-bound, so it is shaped around HBM, not the matrix cores.
//
// A workgroup owns 128 ws columns (for SwiGLU: 64 gate rows + the 64 matching up rows, i.e. one q4/q8 tile record
// row-block each) and walks the whole K. Its 8 waves are 2 column halves x 4 K-slices. Lane l of a wave owns ONE
// weight row: per 32-k (q4, f16) or 64-k (q8) unit it issues one 128-bit load of that row's codes (a wave reads a
// whole 1 KB / 4 KB record row-block, coalesced) plus the row's scale word, decodes them in registers to fp16 pairs,
// and accumulates v_dot2_f32_f16 against X' broadcast from LDS. So every lane has its own sum and no cross-lane
// reduction is needed inside the K loop; the 4 K-slices meet once in LDS at the end.
//
// X' (the prologue applied, rounded to fp16, gemm.js:60-67) is staged per 512-k chunk in LDS by the whole workgroup,
// in the pair order of the weight encoding. The weight loads of chunk c+1 are issued before chunk c is computed.
#include "p0k_device.h"
#include "p0k_launch.h"

namespace p0k {

constexpr int GV_NT = 512, GV_SUB = 4, GV_KC = 512;

template <int WE>
struct Unit;
template <>
struct Unit<W_Q4> { static constexpr int UK = 32; u32x4 code; uint32_t sm; };
template <>
struct Unit<W_Q8> { static constexpr int UK = 64; u32x4 code[4]; uint32_t s; };
template <>
struct Unit<W_F16> { static constexpr int UK = 32; u32x4 v[4]; };

template <int WE, int XM, int MT>
__global__ __launch_bounds__(GV_NT) void k_gemv(Params p) {
  constexpr int UK = Unit<WE>::UK;
  constexpr int UPW = (GV_KC / UK) / GV_SUB;          // units per wave per chunk
  __shared__ __attribute__((aligned(16))) f16 sX[MT * GV_KC];
  __shared__ __attribute__((aligned(16))) float sR[GV_SUB * MT * 128];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ch = wave / GV_SUB, sub = wave % GV_SUB;
  const uint32_t nB = blockIdx.x * 128u;
  const uint32_t r = wrow(p, nB + ch * 64 + lane);

  auto load = [&](Unit<WE> &u, uint32_t k) {
    const uint32_t kc = p.wk0 + k;
    if constexpr (WE == W_Q4) {
      const uint8_t *rec = p.W + ((size_t)(r >> 6) * p.wG + (kc >> 5)) * 1280u;
      u.code = *(const u32x4 *)(rec + (r & 63u) * 16u);
      u.sm = *(const uint32_t *)(rec + 1024u + (r & 63u) * 4u);
    } else if constexpr (WE == W_Q8) {
      const uint8_t *rec = p.W + ((size_t)(r >> 6) * p.wG + (kc >> 6)) * 4224u;
#pragma unroll
      for (int i = 0; i < 4; i++) u.code[i] = *(const u32x4 *)(rec + (r & 63u) * 64u + 16u * i);
      u.s = *(const uint32_t *)(rec + 4096u + (r & 62u) * 2u);
    } else {
      const uint8_t *src = p.W + ((size_t)r * p.wG + kc) * 2;
      if (p.flags & F_WALIGN8) {
#pragma unroll
        for (int i = 0; i < 4; i++) u.v[i] = *(const u32x4 *)(src + 16 * i);
      } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          u32x2 lo = *(const u32x2 *)(src + 16 * i), hi = *(const u32x2 *)(src + 16 * i + 8);
          u.v[i] = (u32x4){lo.x, lo.y, hi.x, hi.y};
        }
      }
    }
  };

  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; m++) acc[m] = 0.0f;

  auto compute = [&](const Unit<WE> &u, int ku) {      // ku: the unit's k offset inside the chunk
    f16x2 w[UK / 2];
    if constexpr (WE == W_Q4) {
      bool fast = q4_fast_ok(u.sm);
      dq_q4_word(u.code.x, u.sm, fast, w + 0);
      dq_q4_word(u.code.y, u.sm, fast, w + 4);
      dq_q4_word(u.code.z, u.sm, fast, w + 8);
      dq_q4_word(u.code.w, u.sm, fast, w + 12);
    } else if constexpr (WE == W_Q8) {
      uint32_t sh = (r & 1u) ? (u.s >> 16) : (u.s & 0xffffu);
      f16x2 s2 = as_h2(sh | (sh << 16));
#pragma unroll
      for (int i = 0; i < 4; i++) {
        dq_q8_word(u.code[i].x, s2, w + 8 * i + 0);
        dq_q8_word(u.code[i].y, s2, w + 8 * i + 2);
        dq_q8_word(u.code[i].z, s2, w + 8 * i + 4);
        dq_q8_word(u.code[i].w, s2, w + 8 * i + 6);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        w[4 * i + 0] = as_h2(u.v[i].x); w[4 * i + 1] = as_h2(u.v[i].y);
        w[4 * i + 2] = as_h2(u.v[i].z); w[4 * i + 3] = as_h2(u.v[i].w);
      }
    }
#pragma unroll
    for (int m = 0; m < MT; m++) {
      const u32x4 *xs = (const u32x4 *)(sX + m * GV_KC + ku);
#pragma unroll
      for (int q = 0; q < UK / 8; q++) {
        u32x4 xv = xs[q];
        acc[m] = __builtin_amdgcn_fdot2(w[4 * q + 0], as_h2(xv.x), acc[m], false);
        acc[m] = __builtin_amdgcn_fdot2(w[4 * q + 1], as_h2(xv.y), acc[m], false);
        acc[m] = __builtin_amdgcn_fdot2(w[4 * q + 2], as_h2(xv.z), acc[m], false);
        acc[m] = __builtin_amdgcn_fdot2(w[4 * q + 3], as_h2(xv.w), acc[m], false);
      }
    }
  };

  Unit<WE> cur[UPW], nxt[UPW];
  const uint32_t K = p.K;
  auto load_chunk = [&](Unit<WE> *dst, uint32_t kc0) {
    uint32_t nu = (K - kc0 < (uint32_t)GV_KC ? K - kc0 : (uint32_t)GV_KC) / UK;
#pragma unroll
    for (int j = 0; j < UPW; j++) {
      uint32_t u = sub + GV_SUB * j;
      if (u < nu) load(dst[j], kc0 + u * UK);
    }
  };

  load_chunk(cur, 0);
  for (uint32_t kc0 = 0; kc0 < K; kc0 += GV_KC) {
    const uint32_t kn = K - kc0 < (uint32_t)GV_KC ? K - kc0 : (uint32_t)GV_KC;
    // X' of this chunk -> LDS
    const uint32_t nb = kn / 8;
    for (uint32_t t = tid; t < MT * nb; t += GV_NT) {
      uint32_t m = t / nb, kb = t - m * nb;
      u32x4 v = (u32x4){0u, 0u, 0u, 0u};
      if (m < p.M) v = xperm<WE>(xload8<XM>(p, m, RowCtx{0, 0, 0}, kc0 + 8 * kb));
      *(u32x4 *)(sX + m * GV_KC + 8 * kb) = v;
    }
    __syncthreads();
    if (kc0 + GV_KC < K) load_chunk(nxt, kc0 + GV_KC);
    const uint32_t nu = kn / UK;
#pragma unroll
    for (int j = 0; j < UPW; j++) {
      uint32_t u = sub + GV_SUB * j;
      if (u < nu) compute(cur[j], u * UK);
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < UPW; j++) cur[j] = nxt[j];
  }

  // the 4 K-slices meet in LDS
#pragma unroll
  for (int m = 0; m < MT; m++) sR[(sub * MT + m) * 128 + ch * 64 + lane] = acc[m];
  __syncthreads();
  for (int t = tid; t < MT * 128; t += GV_NT) {
    float s = sR[t];
#pragma unroll
    for (int q = 1; q < GV_SUB; q++) s += sR[q * MT * 128 + t];
    sR[t] = s;
  }
  __syncthreads();
  epilogue<GV_NT>(p, sR, 128, MT, 0u, nB, tid);
}

template <int WE, int XM, int MT>
static hipError_t launch3(const Params &p, hipStream_t s) {
  dim3 grid((p.N + 127) / 128);
  hipLaunchKernelGGL((k_gemv<WE, XM, MT>), grid, dim3(GV_NT), 0, s, p);
  return hipGetLastError();
}
template <int WE, int XM>
static hipError_t launch2(const Params &p, hipStream_t s) {
  if (p.M <= 1) return launch3<WE, XM, 1>(p, s);
  if (p.M <= 2) return launch3<WE, XM, 2>(p, s);
  if (p.M <= 4) return launch3<WE, XM, 4>(p, s);
  if (p.M <= 8) return launch3<WE, XM, 8>(p, s);
  return launch3<WE, XM, 16>(p, s);
}
template <int WE>
static hipError_t launch1(const Params &p, int xm, hipStream_t s) {
  switch (xm) {
  case X_F16: return launch2<WE, X_F16>(p, s);
  case X_LNMOD: return launch2<WE, X_LNMOD>(p, s);
  case X_RMS: return launch2<WE, X_RMS>(p, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemv(const Params &p, int we, int xm, hipStream_t s) {
  if (p.M > (uint32_t)GEMV_MAX_M) return hipErrorInvalidValue;
  switch (we) {
  case W_Q4: return launch1<W_Q4>(p, xm, s);
  case W_Q8: return launch1<W_Q8>(p, xm, s);
  case W_F16: return launch1<W_F16>(p, xm, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace p0k
