/* p0k_probe.h — C ABI of libp0k_probe.so, the benchmark's measurement kernels (no counterpart in the reference, not
 * part of the gemm path; only bench.py loads it). Each call enqueues on the stream of a libp0k context
 * (p0k_ctx_stream), so the probes time and graph-capture like the gemm calls they are compared with. Returns P0K_OK or
 * a P0K_E_* code; p0kprobe_last_error() gives the message. */
#ifndef P0K_PROBE_H
#define P0K_PROBE_H
#include <stdint.h>

#include "../../include/p0k.h"

#ifdef __cplusplus
extern "C" {
#endif

const char *p0kprobe_last_error(void);
/* the HBM read ceiling: reads `bytes` (below 4 GiB) of a 16-byte aligned device buffer with `blocks` workgroups of
 * `threads` (256 or 512) threads (blocks 0 = 7/8 of the CUs, the decode GEMV's grid for 28672 weight rows; at most
 * ceil(bytes / (threads * 128)) and 65536), 16-byte loads, eight in flight per lane, nothing stored (sink: 4 live
 * device bytes the kernel may write) */
int p0kprobe_stream_read(p0k_ctx *ctx, const void *buf, uint64_t bytes, uint32_t *sink, uint32_t blocks, uint32_t threads);
/* the matrix-core issue ceiling: one 256-thread workgroup per CU per wave per SIMD (waves_per_simd 1 or 2), `iters`
 * iterations of 8 independent 32x32x16 fp16 MFMAs each followed by valu_per_mfma (even, 0..12) independent
 * packed-fp16 FMAs; FLOPs = 32768 * 8 * iters * 4 * CUs * waves_per_simd. random_operands = 0: sparse constant
 * operands (the issue rate alone); 1: pseudo-random fp16 operands (the rate the matrix cores hold on real data) */
int p0kprobe_mfma_valu(p0k_ctx *ctx, int valu_per_mfma, int waves_per_simd, int iters, int random_operands, float *sink);
/* the LDS read ceiling: one workgroup of `waves` (4, 8 or 16) waves per CU, each lane `iters` (1..2^24) x 16
 * conflict-free 16-byte LDS reads; bytes per CU = waves * 16384 * iters. clk: 32 * waves * CUs device bytes receiving,
 * per wave (workgroup-major), the shader clock and the 100 MHz reference clock before and after its loop (uint64:
 * clock start, clock end, reference start, reference end) */
int p0kprobe_lds_read(p0k_ctx *ctx, int waves, int iters, uint64_t *clk);
/* the launch gate: one wave that waits `microseconds` (at most 100000) on the reference clock, so that work the host
 * enqueues behind it starts back to back (sink: 4 live device bytes the kernel may write) */
int p0kprobe_gate(p0k_ctx *ctx, uint32_t microseconds, uint32_t *sink);

#ifdef __cplusplus
}
#endif
#endif /* P0K_PROBE_H */
