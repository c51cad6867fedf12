// p0k_rowstats.hip — per-row (mean, rstd) of an fp32 matrix, the feed of the rms / lnmod prologues.
// Restates src/ops/misc.js:16-44: mode 0 (LayerNorm) mean = sum/cols, var = sum((x-mean)^2)/cols (exact two-pass);
// mode 1 (RMSNorm) mean = 0, var = sum(x^2)/cols; rstd = 1/sqrt(var + eps); ST[(off+row)*2] = (mean, rstd).
// One 256-thread workgroup per row; the row is read once per pass with 16-byte loads when aligned (HBM-bound).
#include "p0k_device.h"
#include "p0k_launch.h"

namespace p0k {

__device__ __forceinline__ float block_sum(float v, float *red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float s = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return s;
}

__global__ __launch_bounds__(256) void k_rowstats(const float *x, uint32_t ld, uint32_t c0, uint32_t cols, int mode,
                                                  float eps, float *st, uint32_t st_off) {
  __shared__ float red[4];
  const uint32_t row = blockIdx.x;
  const float *xr = x + (size_t)row * ld + c0;
  const bool vec = ((((uintptr_t)xr) & 15u) == 0) && (cols % 4u == 0);
  float mean = 0.0f;
  if (mode == 0) {
    float s = 0.0f;
    if (vec) {
      for (uint32_t i = threadIdx.x; i < cols / 4; i += 256) { f32x4 v = ((const f32x4 *)xr)[i]; s += (v.x + v.y) + (v.z + v.w); }
    } else {
      for (uint32_t i = threadIdx.x; i < cols; i += 256) s += xr[i];
    }
    mean = block_sum(s, red) / (float)cols;
  }
  float q = 0.0f;
  if (vec) {
    for (uint32_t i = threadIdx.x; i < cols / 4; i += 256) {
      f32x4 v = ((const f32x4 *)xr)[i] - mean;
      q += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
    }
  } else {
    for (uint32_t i = threadIdx.x; i < cols; i += 256) { float d = xr[i] - mean; q += d * d; }
  }
  float var = block_sum(q, red) / (float)cols;
  if (threadIdx.x == 0) {
    st[(size_t)(st_off + row) * 2] = mean;
    st[(size_t)(st_off + row) * 2 + 1] = __frsqrt_rn(var + eps);
  }
}

hipError_t launch_rowstats(const void *x, uint32_t ld, uint32_t c0, uint32_t rows, uint32_t cols, int mode, float eps,
                           float *st, uint32_t st_off, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(k_rowstats, dim3(rows), dim3(256), 0, s, (const float *)x, ld, c0, cols, mode, eps, st, st_off);
  return hipGetLastError();
}

}  // namespace p0k
