// p0k_stats.hip — the statistics the convolution prologues read: PixelNorm scales (conv3 `pn`) and GroupNorm(32)
// affine coefficients (conv `gn`). Both are HBM-bound reductions over HWC / THWC fp16 activations.
//
//  pixstats  (src/ops/video.js:301-321): R[ro + v] = 1 / sqrt(sum_c x[v][c]^2 / C + eps), one value per voxel.
//            A group of 16 lanes owns one voxel and reads its C channels as 16-byte chunks, so a wave reads four whole
//            voxels per step; the 16 partial sums meet through shuffles.
//  GroupNorm (src/ops/misc.js:50-109): exact two-pass statistics per chunk of 64 pixels, written as partial rows
//            [chunk][group] = (n, mean, M2, 0) (the reference's layout, so partials of several calls - bands of one
//            tensor - merge), then Chan's parallel formula merges the rows: a[c] = gamma[c] / sqrt(M2 / n + eps),
//            b[c] = beta[c] - mean * a[c], so GN(x) = a x + b. The merge runs one workgroup per group; each thread
//            merges a strided subset of rows in order and the 256 partial states meet in a fixed tree, so the result
//            does not depend on timing.
#include "p0k_device.h"
#include "p0k_launch.h"

namespace p0k {

// ------------------------------------------------------------------------------------------------------------ pixstats
__global__ __launch_bounds__(256) void k_pixstats(const uint8_t *x, uint32_t V, uint32_t C, float eps, float *r) {
  const uint32_t g = threadIdx.x & 15;
  const uint32_t v = (blockIdx.x * 256u + threadIdx.x) >> 4;
  const bool live = v < V;
  const uint16_t *row = (const uint16_t *)x + (size_t)(live ? v : 0u) * C;
  float s = 0.0f;
  if (live) {
    const uint32_t c8 = C / 8;
    if ((((uintptr_t)row) & 15u) == 0) {
      for (uint32_t i = g; i < c8; i += 16) {
        const u32x4 w = ((const u32x4 *)row)[i];
        const f16x2 a = as_h2(w.x), b = as_h2(w.y), c = as_h2(w.z), d = as_h2(w.w);
        s += ((float)a.x * (float)a.x + (float)a.y * (float)a.y) + ((float)b.x * (float)b.x + (float)b.y * (float)b.y) +
             ((float)c.x * (float)c.x + (float)c.y * (float)c.y) + ((float)d.x * (float)d.x + (float)d.y * (float)d.y);
      }
      for (uint32_t c = c8 * 8 + g; c < C; c += 16) { const float t = h_val(row[c]); s += t * t; }
    } else {
      for (uint32_t c = g; c < C; c += 16) { const float t = h_val(row[c]); s += t * t; }
    }
  }
  s = sum16(s);
  if (live && g == 0) r[v] = __frsqrt_rn(s / (float)C + eps);
}

hipError_t launch_pixstats(const void *x, uint32_t V, uint32_t C, float eps, float *r, hipStream_t s) {
  if (V == 0) return hipSuccess;
  const uint32_t blocks = (V + 15) / 16;
  hipLaunchKernelGGL(k_pixstats, dim3(blocks), dim3(256), 0, s, (const uint8_t *)x, V, C, eps, r);
  return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------------------ GroupNorm
constexpr uint32_t GN_PIX = 64;   // pixels per partial row (the reference's chunk, so partial buffers interoperate)

// One workgroup per chunk of 64 pixels: thread t owns channel slots t, t + 256 (C <= 512) and sums them over the
// chunk's pixels; the group means come from the per-channel sums, then the same walk sums squared deviations.
__global__ __launch_bounds__(256) void k_gn_partial(const uint16_t *x, uint32_t pix, uint32_t C, f32x4 *part,
                                                    uint32_t wg_off) {
  __shared__ float ch_sum[512];
  __shared__ float g_mean[32];
  const uint32_t t = threadIdx.x, wg = blockIdx.x;
  const uint32_t px0 = wg * GN_PIX, npx = pix - px0 < GN_PIX ? pix - px0 : GN_PIX;
  const uint32_t cpg = C / 32;
  const uint16_t *base = x + (size_t)px0 * C;
  // channel slots of this thread: c = t (and t + 256 when C = 512); for C < 256 several threads share a channel
  float s0 = 0.0f, s1 = 0.0f;
  const uint32_t n = npx * C;
  for (uint32_t e = t; e < n; e += 256) {
    const float v = h_val(base[e]);
    if (C <= 256 || ((e >> 8) & 1u) == 0) s0 += v; else s1 += v;
  }
  ch_sum[t] = s0;
  ch_sum[t + 256] = s1;
  __syncthreads();
  const float cnt = (float)(npx * cpg);
  if (t < 32) {
    // slot j holds channel j % C for j < 256 (C <= 256) or channel j (C = 512)
    float gs = 0.0f;
    for (uint32_t j = 0; j < 512; j++)
      if ((j % C) / cpg == t) gs += ch_sum[j];
    g_mean[t] = gs / fmaxf(cnt, 1.0f);
  }
  __syncthreads();
  s0 = 0.0f; s1 = 0.0f;
  for (uint32_t e = t; e < n; e += 256) {
    const float d = h_val(base[e]) - g_mean[(e % C) / cpg];
    if (C <= 256 || ((e >> 8) & 1u) == 0) s0 += d * d; else s1 += d * d;
  }
  __syncthreads();
  ch_sum[t] = s0;
  ch_sum[t + 256] = s1;
  __syncthreads();
  if (t < 32) {
    float m2 = 0.0f;
    for (uint32_t j = 0; j < 512; j++)
      if ((j % C) / cpg == t) m2 += ch_sum[j];
    part[(size_t)(wg_off + wg) * 32 + t] = (f32x4){cnt, g_mean[t], m2, 0.0f};
  }
}

struct GnState { float n, mean, m2; };
__device__ __forceinline__ GnState gn_merge(GnState a, GnState b) {
  if (b.n <= 0.0f) return a;
  if (a.n <= 0.0f) return b;
  const float nn = a.n + b.n, d = b.mean - a.mean;
  return GnState{nn, a.mean + d * (b.n / nn), a.m2 + b.m2 + d * d * (a.n * b.n / nn)};
}

// One workgroup per group: merge the partial rows, then write the affine coefficients of the group's channels.
__global__ __launch_bounds__(256) void k_gn_finalize(const f32x4 *part, uint32_t nwg, uint32_t C, float eps,
                                                     const float *gamma, const float *beta, float *ab) {
  __shared__ float sn[256], sm[256], sq[256];
  const uint32_t g = blockIdx.x, t = threadIdx.x;
  GnState st{0.0f, 0.0f, 0.0f};
  for (uint32_t w = t; w < nwg; w += 256) {
    const f32x4 q = part[(size_t)w * 32 + g];
    st = gn_merge(st, GnState{q.x, q.y, q.z});
  }
  sn[t] = st.n; sm[t] = st.mean; sq[t] = st.m2;
  __syncthreads();
  for (uint32_t h = 128; h > 0; h >>= 1) {
    if (t < h) {
      const GnState m = gn_merge(GnState{sn[t], sm[t], sq[t]}, GnState{sn[t + h], sm[t + h], sq[t + h]});
      sn[t] = m.n; sm[t] = m.mean; sq[t] = m.m2;
    }
    __syncthreads();
  }
  const float rs = __frsqrt_rn(sq[0] / fmaxf(sn[0], 1.0f) + eps), mean = sm[0];
  const uint32_t cpg = C / 32;
  for (uint32_t c = g * cpg + t; c < (g + 1) * cpg; c += 256) {
    const float a = gamma[c] * rs;
    ab[c] = a;
    ab[C + c] = beta[c] - mean * a;
  }
}

hipError_t launch_gn_partial(const void *x, uint32_t pix, uint32_t C, float *part, uint32_t wg_off, hipStream_t s) {
  if (pix == 0) return hipSuccess;
  hipLaunchKernelGGL(k_gn_partial, dim3((pix + GN_PIX - 1) / GN_PIX), dim3(256), 0, s, (const uint16_t *)x, pix, C,
                     (f32x4 *)part, wg_off);
  return hipGetLastError();
}

hipError_t launch_gn_finalize(const float *part, uint32_t nwg, uint32_t C, float eps, const float *gamma,
                              const float *beta, float *ab, hipStream_t s) {
  hipLaunchKernelGGL(k_gn_finalize, dim3(32), dim3(256), 0, s, (const f32x4 *)part, nwg, C, eps, gamma, beta, ab);
  return hipGetLastError();
}

}  // namespace p0k
