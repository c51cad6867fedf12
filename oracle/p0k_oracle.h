/* p0k_oracle.h — CPU restatement of the reference's `gemm` path. TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker the parity tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the HIP
 * kernels against. The product (libp0k.so and the Node shim) never links, loads or calls it.
 *
 * It takes the same p0k_gemm_args as the HIP library, with HOST pointers in place of device buffers, and writes Y the
 * way the reference kernel does (src/ops/gemm.js), accumulating in float64 like the reference's cpuGemm
 * (test/kernels.test.js:29). The fp16 rounding points of the reference kernel are reproduced: X' after the prologue
 * (gemm.js:62-91), the dequantised weight (gemm.js:152,163,169), and the single rounding of the epilogue result.
 */
#ifndef P0K_ORACLE_H
#define P0K_ORACLE_H
#include <stdint.h>
#include "../include/p0k.h"

#ifdef __cplusplus
extern "C" {
#endif

uint16_t or_f2h(float v);                 /* src/core/gpu.js:276-291: fp32 -> fp16, round to nearest even */
float or_h2f(uint16_t h);                 /* src/core/gpu.js:292-297 */
float or_rf16(float v);                   /* h2f(f2h(v)), src/convert/encode.js:12 */
float or_rhe(float v);                    /* round half to even, src/convert/encode.js:13 */

/* encoders, src/convert/encode.js:56-95; deq (optional) receives the fp32 dequantised weights; 0 or -1 (bad shape) */
int or_pack_q4(const float *W, int rows, int K, uint8_t *out, float *deq);
int or_pack_q8(const float *W, int rows, int K, uint8_t *out, float *deq);
void or_pack_f16(const float *W, int64_t n, uint16_t *out);
int64_t or_tensor_bytes(int enc, int rows, int cols);

/* the fp16 weight the kernel multiplies by: W'(row r, column kc) of an encoded tensor (FORMAT.md layouts) */
uint16_t or_weight_f16(int enc, const uint8_t *w, uint32_t wG, uint32_t r, uint32_t kc);
/* decode a whole tensor to fp16 [rows][cols] (q4/q8; wG = cols/32 or cols/64) */
void or_dequant(int enc, const uint8_t *w, int rows, int cols, uint16_t *out);

/* test-suite data generators, test/kernels.test.js:12-13 (xorshift32 + Box-Muller) */
void or_randn(float *out, int64_t n, uint32_t seed, double scale);
void or_rand_uniform(float *out, int64_t n, uint32_t seed, float lo, float hi);

/* which dequantised weights or_gemm multiplies by: 0 = fp16-rounded (the reference kernel, gemm.js:152,163; default),
 * 1 = fp32 (the reference test suite's cpuGemm over the encoders' deq output, test/kernels.test.js:25-29) */
void or_set_weight_model(int model);
/* rows [m0, m1) of one gemm call (src/ops/gemm.js semantics), all buffers on the host; returns 0 or -1 (bad args) */
int or_gemm(const p0k_gemm_args *a, uint32_t m0, uint32_t m1);
/* src/ops/misc.js:16-44 */
int or_rowstats(const p0k_rowstats_args *a);

/* the test suite's plain CPU references (test/kernels.test.js:29, :52-65), fp64 accumulation */
void or_cpu_gemm(const float *X, const float *W, int M, int N, int K, float *Y);
void or_cpu_conv3(const float *X, const float *Wt, int T, int H, int W, int C, int N, float *Y);
/* pixstats / GroupNorm statistics (src/ops/video.js:301-321, src/ops/misc.js:50-109) */
void or_pixstats(const uint16_t *x, uint32_t V, uint32_t C, float eps, float *r);
void or_gn_partial(const uint16_t *x, uint32_t pix, uint32_t C, float *part);
void or_gn_finalize(const float *part, uint32_t nwg, uint32_t C, float eps, const float *gamma, const float *beta,
                    float *ab);
/* attention, head size 128 (cpuAttn, test/kernels.test.js:30-49) */
void or_attention(const uint16_t *Q, const uint16_t *K, const uint16_t *V, uint16_t *O, uint32_t Lq, uint32_t Lk,
                  uint32_t Hq, uint32_t Hkv, uint32_t ldo, uint32_t mode, uint32_t nvalid, float scale, float cap);

#ifdef __cplusplus
}
#endif
#endif
