// p0k_probe.hip — measurement kernels of the benchmark, not part of the gemm path and not in libp0k.so: they are
// built into libp0k_probe.so, which only bench.py loads (C ABI in p0k_probe.h).
//
// HBM read ceiling: a plain streaming read of a buffer, by default with the GEMV's launch shape (one 512-thread
// workgroup per 128-column tile's worth of bytes, 16-byte non-temporal loads, eight in flight per lane; 256-thread
// workgroups and any grid size are selectable), nothing computed and nothing stored. Its time per call, in the same
// graph-replay timing as the bench, is the fastest a kernel can move that many bytes from HBM in one launch. The
// loads are the decode's own streaming form (sload128: buffer loads, sc0 nt).
#include "../csrc/p0k_device.h"
#include "p0k_probe.h"

#include <algorithm>
#include <cstdio>

namespace p0k {

template <int NT>
__global__ __launch_bounds__(NT) void k_stream_read(const u32x4 *p, uint32_t n, uint32_t *sink) {
  constexpr int U = 8;
  // n < 2^28 16-byte words (32-bit byte offsets) and gridDim.x * NT * U <= n + NT * U (both checked on the host), so
  // neither the start nor the stride wraps; the loop index is 64-bit all the same
  uint64_t i = (uint64_t)blockIdx.x * (NT * U) + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * (NT * U);
  const srsrc r = stream_rsrc((const uint8_t *)p);
  uint32_t acc = 0;
  for (; i < n; i += stride) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint64_t j = i + (uint64_t)u * NT;
      v[u] = j < n ? sload128(r, (uint32_t)j * 16u) : (u32x4){0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9e3779b9u) *sink = acc;      // keeps the loads; practically never taken
}

hipError_t launch_probe_stream(const void *buf, uint64_t bytes, uint32_t *sink, unsigned blocks, unsigned threads,
                                     hipStream_t s) {
  if (bytes < 16) return hipSuccess;
  const uint32_t n = (uint32_t)(bytes / 16);
  if (threads == 256) hipLaunchKernelGGL(k_stream_read<256>, dim3(blocks), dim3(256), 0, s, (const u32x4 *)buf, n, sink);
  else hipLaunchKernelGGL(k_stream_read<512>, dim3(blocks), dim3(512), 0, s, (const u32x4 *)buf, n, sink);
  return hipGetLastError();
}

}  // namespace p0k

namespace p0k {

// The matrix-core issue ceiling of the GEMM kernels: every iteration issues 8 independent v_mfma_f32_32x32x16_f16 on
// eight accumulators and V independent packed-fp16 FMAs per MFMA, interleaved one MFMA then V VALU (the GEMM loop's
// sched_group_barrier pattern). FLOP rate against the 2.5 PFLOP/s peak, for V = 0 .. 12 and one or two waves per SIMD,
// says how much decode work per MFMA the loop can hide.
// RND = 0: sparse constant operands (one non-zero per fragment, the issue rate alone); RND = 1: every operand a
// distinct pseudo-random fp16 in (-2, 2) per lane and accumulator, as a GEMM on real data feeds the matrix cores
// (their power draw, and with it the clock the part holds, depends on the operand bits).
template <int V, int RND>
__global__ __launch_bounds__(256) void k_mfma_valu(float *sink, int iters) {
  f32x16 acc[8];
#pragma unroll
  for (int i = 0; i < 8; i++) acc[i] = (f32x16){};
  f16x8 a[8], b[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    a[i] = (f16x8){};
    b[i] = (f16x8){};
    if (RND) {
      uint32_t h = (threadIdx.x + 1u) * 2654435761u ^ (uint32_t)(i + 1) * 40503u;
#pragma unroll
      for (int q = 0; q < 8; q++) {
        h = h * 1664525u + 1013904223u;
        a[i][q] = (f16)((float)(int)(h >> 16 & 0xffffu) * (1.0f / 16384.0f) - 2.0f);
        h = h * 1664525u + 1013904223u;
        b[i][q] = (f16)((float)(int)(h >> 16 & 0xffffu) * (1.0f / 16384.0f) - 2.0f);
      }
    } else {
      a[i][0] = (f16)(float)(threadIdx.x & 7);
      b[i][1] = (f16)1.0f;
    }
  }
  f16x2 v[16];
#pragma unroll
  for (int i = 0; i < 16; i++) v[i] = (f16x2){(f16)(float)(i + (threadIdx.x & 3)), (f16)1.0f};
  const f16x2 m = {(f16)0.999f, (f16)0.999f}, c = {(f16)0.001f, (f16)0.001f};
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[i], acc[i], 0, 0, 0);
#pragma unroll
    for (int q = 0; q < 8 * V; q++) v[q % 16] = __builtin_elementwise_fma(v[q % 16], m, c);
#pragma unroll
    for (int q = 0; q < 8; q++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (V) __builtin_amdgcn_sched_group_barrier(0x002, V, 0);
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) s += acc[i][0] + acc[i][15];
#pragma unroll
  for (int i = 0; i < 16; i++) s += (float)v[i].x;
  if (s == 1.2345f) *sink = s;              // keeps the work; practically never taken
}

template <int RND>
static hipError_t launch_mfma_valu_r(int valu_per_mfma, unsigned blocks, int iters, float *sink, hipStream_t s) {
  switch (valu_per_mfma) {
  case 0: hipLaunchKernelGGL((k_mfma_valu<0, RND>), dim3(blocks), dim3(256), 0, s, sink, iters); break;
  case 2: hipLaunchKernelGGL((k_mfma_valu<2, RND>), dim3(blocks), dim3(256), 0, s, sink, iters); break;
  case 4: hipLaunchKernelGGL((k_mfma_valu<4, RND>), dim3(blocks), dim3(256), 0, s, sink, iters); break;
  case 6: hipLaunchKernelGGL((k_mfma_valu<6, RND>), dim3(blocks), dim3(256), 0, s, sink, iters); break;
  case 8: hipLaunchKernelGGL((k_mfma_valu<8, RND>), dim3(blocks), dim3(256), 0, s, sink, iters); break;
  case 10: hipLaunchKernelGGL((k_mfma_valu<10, RND>), dim3(blocks), dim3(256), 0, s, sink, iters); break;
  case 12: hipLaunchKernelGGL((k_mfma_valu<12, RND>), dim3(blocks), dim3(256), 0, s, sink, iters); break;
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_probe_mfma(int valu_per_mfma, int random_operands, unsigned blocks, int iters, float *sink, hipStream_t s) {
  return random_operands ? launch_mfma_valu_r<1>(valu_per_mfma, blocks, iters, sink, s)
                         : launch_mfma_valu_r<0>(valu_per_mfma, blocks, iters, sink, s);
}

}  // namespace p0k

namespace p0k {

// The LDS read ceiling: one workgroup of W waves per CU, every lane reading 16 bytes per ds_read_b128 from a 64 KB
// array, 16 reads per iteration, each wave's 64 lanes one contiguous KB (no bank conflicts), the GEMM loops' fragment
// read. Every wave writes the shader clock (s_memtime) and the 100 MHz reference clock (s_memrealtime) before and
// after its loop to clk[4 (block W + wave) ..], so the host gets both the bytes per clock of a CU and the clock the
// part ran at.
template <int W>
__global__ __launch_bounds__(64 * W) void k_lds_read(uint64_t *clk, int iters) {
  __shared__ u32x4 s[4096];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  for (int i = tid; i < 4096; i += 64 * W) s[i] = (u32x4){(uint32_t)i, 1u, 2u, 3u};
  __syncthreads();
  u32x4 acc = {0u, 0u, 0u, 0u};
  const uint64_t c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (uint32_t it = 0; it < (uint32_t)iters; it++) {
#pragma unroll
    for (uint32_t j = 0; j < 16; j++) acc += s[((it * 16u + j) * 64u + lane + wv * 128u) & 4095u];
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  const uint64_t c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  if (lane == 0) {
    uint64_t *o = clk + 4 * ((size_t)blockIdx.x * W + wv);
    o[0] = c0;
    o[1] = c1;
    o[2] = r0;
    o[3] = r1 + (acc.x == 0x9e3779b9u ? acc.y : 0u);    // keeps the reads; practically never changes the value
  }
}

hipError_t launch_probe_lds(int waves, unsigned blocks, int iters, uint64_t *clk, hipStream_t s) {
  switch (waves) {
  case 4: hipLaunchKernelGGL(k_lds_read<4>, dim3(blocks), dim3(256), 0, s, clk, iters); break;
  case 8: hipLaunchKernelGGL(k_lds_read<8>, dim3(blocks), dim3(512), 0, s, clk, iters); break;
  case 16: hipLaunchKernelGGL(k_lds_read<16>, dim3(blocks), dim3(1024), 0, s, clk, iters); break;
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace p0k

namespace p0k {

// The launch gate of the benchmark's timed regions: one wave that waits on the 100 MHz reference clock for `ticks`
// ticks (at most max_iters sleeps of about 64 clocks each, so it always ends), enqueued right before the first timing
// event. While it runs the host enqueues the timed graph behind it, so the timed calls start back to back instead of
// behind the host's own launch latency (the blocking-kernel practice of GPU benchmark harnesses).
__global__ __launch_bounds__(64) void k_gate(uint64_t ticks, uint32_t max_iters, uint32_t *sink) {
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  uint32_t it = 0;
  while (__builtin_amdgcn_s_memrealtime() - t0 < ticks && it < max_iters) {
    __builtin_amdgcn_s_sleep(1);
    it++;
  }
  if (it == 0xffffffffu && threadIdx.x == 0) *sink = it;   // never taken; keeps the loop
}

}  // namespace p0k

// ------------------------------------------------------------------------------------------------ C ABI
namespace {
thread_local char g_perr[256];
int perr(int code, const char *msg) {
  snprintf(g_perr, sizeof g_perr, "%s", msg);
  return code;
}
int hperr(hipError_t e, const char *what) {
  snprintf(g_perr, sizeof g_perr, "%s: %s", what, hipGetErrorName(e));
  return P0K_E_HIP;
}
hipStream_t stream_of(p0k_ctx *c) { return (hipStream_t)p0k_ctx_stream(c); }
}  // namespace

extern "C" {

const char *p0kprobe_last_error(void) { return g_perr; }

int p0kprobe_stream_read(p0k_ctx *c, const void *buf, uint64_t bytes, uint32_t *sink, uint32_t blocks, uint32_t threads) {
  // the arguments are checked before the context is used, so a refusal never touches the GPU
  if (!buf || !sink) return perr(P0K_E_ARG, "stream_read: NULL argument");
  if (((uintptr_t)buf & 15u) != 0) return perr(P0K_E_ARG, "stream_read: buf must be 16-byte aligned");
  if (threads != 256 && threads != 512) return perr(P0K_E_ARG, "stream_read: threads must be 256 or 512");
  if (bytes >= (1ull << 32)) return perr(P0K_E_ARG, "stream_read: bytes must be below 4 GiB");
  // every workgroup must own at least one 16-byte word of its first pass: more would only add idle workgroups, and
  // the grid stays far below where the stride could wrap
  const uint64_t max_blocks = bytes / ((uint64_t)threads * 8u * 16u) + 1u;
  if (blocks > max_blocks || blocks > 65536u)
    return perr(P0K_E_ARG, "stream_read: blocks above bytes / (threads * 128) + 1 or 65536");
  if (!c) return perr(P0K_E_ARG, "stream_read: NULL context");
  if (!blocks) blocks = std::min<uint32_t>((uint32_t)p0k_ctx_cus(c) * 7u / 8u, (uint32_t)max_blocks);
  hipError_t e = p0k::launch_probe_stream(buf, bytes, sink, blocks, threads, stream_of(c));
  return e == hipSuccess ? P0K_OK : hperr(e, "stream_read launch");
}

int p0kprobe_mfma_valu(p0k_ctx *c, int valu_per_mfma, int waves_per_simd, int iters, int random_operands, float *sink) {
  if (!c || !sink) return perr(P0K_E_ARG, "mfma_valu: NULL argument");
  if (waves_per_simd < 1 || waves_per_simd > 2 || iters < 1 || valu_per_mfma < 0 || valu_per_mfma > 12 || valu_per_mfma % 2)
    return perr(P0K_E_ARG, "mfma_valu: waves_per_simd 1 or 2, iters > 0, valu_per_mfma even in 0..12");
  hipError_t e = p0k::launch_probe_mfma(valu_per_mfma, random_operands != 0, (unsigned)p0k_ctx_cus(c) * (unsigned)waves_per_simd,
                                   iters, sink, stream_of(c));
  return e == hipSuccess ? P0K_OK : hperr(e, "mfma_valu launch");
}

int p0kprobe_lds_read(p0k_ctx *c, int waves, int iters, uint64_t *clk) {
  if (!c || !clk) return perr(P0K_E_ARG, "lds_read: NULL argument");
  if ((waves != 4 && waves != 8 && waves != 16) || iters < 1 || iters > (1 << 24))
    return perr(P0K_E_ARG, "lds_read: waves 4, 8 or 16, iters in 1..2^24");
  hipError_t e = p0k::launch_probe_lds(waves, (unsigned)p0k_ctx_cus(c), iters, clk, stream_of(c));
  return e == hipSuccess ? P0K_OK : hperr(e, "lds_read launch");
}

int p0kprobe_gate(p0k_ctx *c, uint32_t microseconds, uint32_t *sink) {
  if (!c || !sink) return perr(P0K_E_ARG, "gate: NULL argument");
  if (microseconds > 100000u) return perr(P0K_E_ARG, "gate: at most 100000 microseconds");
  // 100 ticks per microsecond; one s_sleep 1 is at least 64 shader clocks (>= 25 ns at 2.4 GHz), so 100 iterations
  // per microsecond bound the loop past the requested time
  hipLaunchKernelGGL(p0k::k_gate, dim3(1), dim3(64), 0, stream_of(c), (uint64_t)microseconds * 100u,
                     microseconds * 100u + 1000u, sink);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? P0K_OK : hperr(e, "gate launch");
}

}  // extern "C"
