// p0k_rowstats.hip — per-row (mean, rstd) of an fp32 matrix, the feed of the rms / lnmod prologues.
// Restates src/ops/misc.js:16-44: mode 0 (LayerNorm) mean = sum/cols, var = sum((x-mean)^2)/cols (exact two-pass);
// mode 1 (RMSNorm) mean = 0, var = sum(x^2)/cols; rstd = 1/sqrt(var + eps); ST[(off+row)*2] = (mean, rstd).
// One 256-thread workgroup per row; the row is read with 16-byte loads when aligned (HBM-bound): once, held in
// registers, for rows of up to 8192 aligned columns, else once per pass.
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

// Rows of at most NV * 1024 aligned columns: each thread loads its NV 16-byte pieces of the row at once (all in flight
// after the launch instead of one round trip per piece) and keeps them in registers for both passes, so the row is read
// from memory once in either mode. The sums run in the same order as k_rowstats (piece i = thread + 256 i ascending),
// so the results are the same bits.
template <int NV>
__global__ __launch_bounds__(256) void k_rowstats_reg(const float *x, uint32_t ld, uint32_t c0, uint32_t cols, int mode,
                                                      float eps, float *st, uint32_t st_off) {
  __shared__ float red[4];
  const uint32_t row = blockIdx.x, n4 = cols / 4u;
  const f32x4 *xr = (const f32x4 *)(x + (size_t)row * ld + c0);
  f32x4 v[NV];
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const uint32_t j = threadIdx.x + 256u * (uint32_t)i;
    v[i] = j < n4 ? xr[j] : (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  }
  float mean = 0.0f;
  if (mode == 0) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++)
      if (threadIdx.x + 256u * (uint32_t)i < n4) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    mean = block_sum(s, red) / (float)cols;
  }
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; i++)
    if (threadIdx.x + 256u * (uint32_t)i < n4) {
      const f32x4 d = v[i] - mean;
      q += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
    }
  const float var = block_sum(q, red) / (float)cols;
  if (threadIdx.x == 0) {
    st[(size_t)(st_off + row) * 2] = mean;
    st[(size_t)(st_off + row) * 2 + 1] = __frsqrt_rn(var + eps);
  }
}

hipError_t launch_rowstats(const void *x, uint32_t ld, uint32_t c0, uint32_t rows, uint32_t cols, int mode, float eps,
                           float *st, uint32_t st_off, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  const float *xf = (const float *)x;
  // the register form needs every row's start 16-byte aligned: the base (with c0) and the pitch
  const bool vec = ((((uintptr_t)(xf + c0)) & 15u) == 0) && (ld % 4u == 0) && (cols % 4u == 0);
  const uint32_t nv = (cols + 1023u) / 1024u;
  if (vec && nv >= 1 && nv <= 8) {
#define RS_CASE(N) case N: hipLaunchKernelGGL(k_rowstats_reg<N>, dim3(rows), dim3(256), 0, s, xf, ld, c0, cols, mode, eps, st, st_off); break;
    switch (nv <= 2 ? 2 : nv <= 4 ? 4 : 8) {
      RS_CASE(2) RS_CASE(4) RS_CASE(8)
    }
#undef RS_CASE
  } else {
    hipLaunchKernelGGL(k_rowstats, dim3(rows), dim3(256), 0, s, xf, ld, c0, cols, mode, eps, st, st_off);
  }
  return hipGetLastError();
}

}  // namespace p0k
