// p0k_launch.h — host-side launchers of the gfx950 kernels (one per kernel family), called by p0k_runtime.cpp.
#pragma once
#include <hip/hip_runtime.h>

namespace p0k {
struct Params;
// MFMA GEMM (any M): 128 x 128 tiles, 256 threads
hipError_t launch_gemm_mfma(const Params &p, int we, int xm, hipStream_t s);
// decode GEMV (M <= 16, prologue f16 / rms / lnmod): 128 ws columns per workgroup, 512 threads
hipError_t launch_gemv(const Params &p, int we, int xm, hipStream_t s);
// rowstats (src/ops/misc.js:16-44)
hipError_t launch_rowstats(const void *x, uint32_t ld, uint32_t c0, uint32_t rows, uint32_t cols, int mode, float eps,
                           float *st, uint32_t st_off, hipStream_t s);
constexpr int GEMV_MAX_M = 16;
}  // namespace p0k
