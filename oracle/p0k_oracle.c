/* p0k_oracle.c — CPU restatement of the reference's `gemm` path. TEST INFRASTRUCTURE ONLY: the parity checker for the
 * HIP library; nothing in the product links it.
 *
 * Each function names the reference lines it restates. Parity pins (tests/test_oracle.py):
 *   or_f2h / or_h2f      all 2^16 fp16 codes round-trip; RNE ties, subnormals, overflow against numpy's float16 cast;
 *                        known answers 1.0 <-> 0x3C00, -2 <-> 0xC000 (test/convert.test.mjs:47)
 *   or_pack_q4 / q8      FORMAT.md closed form (record sizes, byte positions), |w - deq| <= s/2, codes in range, the
 *                        calibrate/bench known-answer scale word (src/core/tune.js:43), brute-force requantisation
 *   or_weight_f16        exhaustive: all 16 q4 codes / 256 q8 codes x sampled scales vs f16(f32(q*s + mn))
 *   or_gemm              plain GEMM against numpy float64 matmul; every prologue / epilogue against an independent
 *                        numpy formulation of the reference formulas, plus invariants (rotation preserves norm, V
 *                        passes unchanged, conv3 chunks == whole clip, conv3 == textbook cross-correlation)
 *   or_rowstats          numpy mean / variance
 *   or_pixstats          src/ops/video.js:301-321 (PixelNorm scale per voxel)
 *   or_gn_partial        src/ops/misc.js:50-76 (per 64-pixel chunk: n, mean, M2 of each of 32 groups)
 *   or_gn_finalize       src/ops/misc.js:77-91 (Chan's merge of the chunks in order; a = gamma rstd, b = beta - mean a)
 *   or_attention         cpuAttn of test/kernels.test.js:30-49 (exact softmax in fp64), rounded to fp16 like the kernel
 */
#include "p0k_oracle.h"

#include <math.h>
#include <stddef.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ fp16 (src/core/gpu.js:276-299) */
uint16_t or_f2h(float v) {
  uint32_t x; memcpy(&x, &v, 4);
  uint32_t sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xffu, man = x & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));      /* inf / quiet NaN */
  int e = (int)exp - 127 + 15;                                                     /* biased fp16 exponent */
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {                                                                    /* fp16 subnormal or zero */
    if (e < -10) return (uint16_t)sign;
    uint32_t full = man | 0x800000u, shift = (uint32_t)(14 - e);
    uint32_t q = full >> shift, rest = full & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rest > half || (rest == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t r = sign | ((uint32_t)e << 10) | (man >> 13), rest = man & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (r & 1u))) r++;                       /* a carry may reach infinity: RNE */
  return (uint16_t)r;
}

float or_h2f(uint16_t h) {
  double s = (h & 0x8000) ? -1.0 : 1.0;
  int e = (h >> 10) & 0x1f, m = h & 0x3ff;
  if (e == 0) return (float)(s * m * 5.960464477539063e-8);
  if (e == 31) return m ? NAN : (float)(s * INFINITY);
  return (float)(s * (1.0 + m / 1024.0) * ldexp(1.0, e - 15));
}

float or_rf16(float v) { return or_h2f(or_f2h(v)); }

float or_rhe(float x) {      /* src/convert/encode.js:13 on an fp32 value */
  double f = floor((double)x), d = (double)x - f;
  if (d > 0.5) return (float)(f + 1);
  if (d < 0.5) return (float)f;
  return (float)(fmod(f, 2.0) == 0.0 ? f : f + 1);
}

/* ------------------------------------------------------------------ encoders (src/convert/encode.js:56-95, FORMAT.md) */
static void put32(uint8_t *p, uint32_t v) { p[0] = v & 255; p[1] = (v >> 8) & 255; p[2] = (v >> 16) & 255; p[3] = v >> 24; }
static uint32_t get32(const uint8_t *p) { return p[0] | (p[1] << 8) | (p[2] << 16) | ((uint32_t)p[3] << 24); }
static uint16_t get16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

int or_pack_q4(const float *W, int rows, int K, uint8_t *out, float *deq) {
  if (rows % 64 || K % 32) return -1;
  int NT = rows / 64, G = K / 32;
  for (int t = 0; t < NT; t++)
    for (int g = 0; g < G; g++) {
      uint8_t *rec = out + ((int64_t)t * G + g) * 1280;
      for (int r = 0; r < 64; r++) {
        int64_t base = (int64_t)(t * 64 + r) * K + (int64_t)g * 32;
        float lo = INFINITY, hi = -INFINITY;
        for (int i = 0; i < 32; i++) { float v = W[base + i]; if (v < lo) lo = v; if (v > hi) hi = v; }
        float mn = or_rf16(lo);
        volatile float span = hi - mn;                 /* fp32 maths, one rounding per operation */
        volatile float sd = span / 15.0f;
        float s = or_rf16(sd);
        if (s == 0.0f) s = 1.0f;
        for (int j = 0; j < 16; j++) {
          int q[2];
          for (int h = 0; h < 2; h++) {
            volatile float dv = W[base + 2 * j + h] - mn;
            volatile float qv = dv / s;
            float rq = or_rhe(qv);
            q[h] = rq < 0 ? 0 : rq > 15 ? 15 : (int)rq;
            if (deq) deq[base + 2 * j + h] = (float)((double)q[h] * s + mn);
          }
          rec[r * 16 + j] = (uint8_t)(q[0] | (q[1] << 4));
        }
        put32(rec + 1024 + r * 4, (uint32_t)or_f2h(s) | ((uint32_t)or_f2h(mn) << 16));
      }
    }
  return 0;
}

int or_pack_q8(const float *W, int rows, int K, uint8_t *out, float *deq) {
  if (rows % 64 || K % 64) return -1;
  int NT = rows / 64, G = K / 64;
  for (int t = 0; t < NT; t++)
    for (int g = 0; g < G; g++) {
      uint8_t *rec = out + ((int64_t)t * G + g) * 4224;
      for (int r = 0; r < 64; r++) {
        int64_t base = (int64_t)(t * 64 + r) * K + (int64_t)g * 64;
        float am = 0.0f;
        for (int i = 0; i < 64; i++) { float a = fabsf(W[base + i]); if (a > am) am = a; }
        volatile float sd = am / 127.0f;
        float s = or_rf16(sd);
        if (s == 0.0f) s = 1.0f;
        for (int i = 0; i < 64; i++) {
          volatile float qv = W[base + i] / s;
          float rq = or_rhe(qv);
          int q = rq < -128 ? -128 : rq > 127 ? 127 : (int)rq;
          rec[r * 64 + i] = (uint8_t)(q & 255);
          if (deq) deq[base + i] = (float)((double)q * s);
        }
        uint16_t sh = or_f2h(s);
        rec[4096 + r * 2] = sh & 255; rec[4096 + r * 2 + 1] = sh >> 8;
      }
    }
  return 0;
}

void or_pack_f16(const float *W, int64_t n, uint16_t *out) {
  for (int64_t i = 0; i < n; i++) out[i] = or_f2h(W[i]);
}

int64_t or_tensor_bytes(int enc, int rows, int cols) {
  if (enc == P0K_ENC_Q4G32A_T64) return (int64_t)(rows / 64) * (cols / 32) * 1280;
  if (enc == P0K_ENC_Q8G64S_T64) return (int64_t)(rows / 64) * (cols / 64) * 4224;
  return (int64_t)rows * cols * 2;
}

/* ------------------------------------------------------------------ dequantisation (gemm.js:143-172, FORMAT.md) */
uint16_t or_weight_f16(int enc, const uint8_t *w, uint32_t wG, uint32_t r, uint32_t kc) {
  if (enc == P0K_ENC_Q4G32A_T64) {
    const uint8_t *rec = w + ((uint64_t)(r >> 6) * wG + kc / 32) * 1280;
    uint32_t rr = r & 63, kk = kc % 32;
    uint32_t code = (rec[rr * 16 + kk / 2] >> ((kk & 1) * 4)) & 15;
    uint32_t sm = get32(rec + 1024 + rr * 4);
    float s = or_h2f((uint16_t)(sm & 0xffff)), mn = or_h2f((uint16_t)(sm >> 16));
    float v = fmaf((float)code, s, mn);        /* q*s is exact in fp32; the one rounding is the add (gemm.js:152) */
    return or_f2h(v);
  }
  if (enc == P0K_ENC_Q8G64S_T64) {
    const uint8_t *rec = w + ((uint64_t)(r >> 6) * wG + kc / 64) * 4224;
    uint32_t rr = r & 63, kk = kc % 64;
    int q = (int8_t)rec[rr * 64 + kk];
    float s = or_h2f(get16(rec + 4096 + rr * 2));
    return or_f2h((float)q * s);               /* gemm.js:162-163 */
  }
  return get16(w + ((uint64_t)r * wG + kc) * 2);
}

void or_dequant(int enc, const uint8_t *w, int rows, int cols, uint16_t *out) {
  uint32_t wG = enc == P0K_ENC_Q4G32A_T64 ? cols / 32 : enc == P0K_ENC_Q8G64S_T64 ? cols / 64 : cols;
  for (int r = 0; r < rows; r++)
    for (int k = 0; k < cols; k++) out[(int64_t)r * cols + k] = or_weight_f16(enc, w, wG, r, k);
}

/* ------------------------------------------------------------------ test data (test/kernels.test.js:12-13) */
typedef struct { uint32_t s; } or_rng;
static double rng_next(or_rng *g) {
  uint32_t s = g->s;
  s ^= s << 13;
  s ^= (uint32_t)(((int32_t)s) >> 17);        /* JS `>>` on the int32 view: arithmetic shift */
  s ^= s << 5;
  g->s = s;
  return s / 4294967296.0;
}

void or_randn(float *out, int64_t n, uint32_t seed, double scale) {
  or_rng g = { seed ? seed : 1u };
  const double PI = 3.141592653589793;
  for (int64_t i = 0; i < n; i += 2) {
    double u = rng_next(&g), v = rng_next(&g);
    if (u < 1e-9) u = 1e-9;
    double m = sqrt(-2.0 * log(u)) * scale;
    out[i] = (float)(m * cos(2 * PI * v));
    if (i + 1 < n) out[i + 1] = (float)(m * sin(2 * PI * v));
  }
}

void or_rand_uniform(float *out, int64_t n, uint32_t seed, float lo, float hi) {
  or_rng g = { seed ? seed : 1u };
  for (int64_t i = 0; i < n; i++) out[i] = (float)(lo + (hi - lo) * rng_next(&g));
}

/* ------------------------------------------------------------------ weight models
 * 0: the reference kernel's: each dequantised weight rounded to fp16 (gemm.js:152,163)
 * 1: the reference test suite's cpuGemm: the encoders' fp32 dequantised weights (src/convert/encode.js:68,85) */
static int g_weight_model = 0;
void or_set_weight_model(int m) { g_weight_model = m; }

static float weight_value(int enc, const uint8_t *w, uint32_t wG, uint32_t r, uint32_t kc) {
  if (g_weight_model == 1 && enc == P0K_ENC_Q4G32A_T64) {
    const uint8_t *rec = w + ((uint64_t)(r >> 6) * wG + kc / 32) * 1280;
    uint32_t rr = r & 63, kk = kc % 32;
    uint32_t code = (rec[rr * 16 + kk / 2] >> ((kk & 1) * 4)) & 15, sm = get32(rec + 1024 + rr * 4);
    return (float)((double)code * or_h2f((uint16_t)(sm & 0xffff)) + or_h2f((uint16_t)(sm >> 16)));
  }
  if (g_weight_model == 1 && enc == P0K_ENC_Q8G64S_T64) {
    const uint8_t *rec = w + ((uint64_t)(r >> 6) * wG + kc / 64) * 4224;
    uint32_t rr = r & 63, kk = kc % 64;
    return (float)((double)(int8_t)rec[rr * 64 + kk] * or_h2f(get16(rec + 4096 + rr * 2)));
  }
  return or_h2f(or_weight_f16(enc, w, wG, r, kc));
}

/* ------------------------------------------------------------------ the GEMM (src/ops/gemm.js) */
typedef struct {
  const p0k_gemm_args *a;
  uint32_t ldx, ldy, wG, Nw, ks, stride, eps_set;
  float eps;
} ocfg;

static float silu(float z) { return z / (1.0f + expf(-z)); }

/* X'[row, k] as the fp16 value the kernel multiplies by (gemm.js:60-95) */
static float xprime(const ocfg *c, uint32_t row, uint32_t k) {
  const p0k_gemm_args *a = c->a;
  const uint8_t *xb = (const uint8_t *)a->x_buf + a->x_off;
  switch (a->x_mode) {
  case P0K_X_F16:
    return or_h2f(get16(xb + ((uint64_t)row * c->ldx + a->x_k0 + k) * 2));
  case P0K_X_RMS: case P0K_X_LNMOD: {
    float x; memcpy(&x, xb + ((uint64_t)row * c->ldx + a->x_k0 + k) * 4, 4);
    const float *st = a->st_buf + (uint64_t)(a->st_off + row) * 2;
    uint32_t kk = a->x_k0 + k;
    if (a->x_mode == P0K_X_RMS) {
      volatile float t = x * st[1];
      return or_rf16(t * a->pv_buf[a->pv_off + kk]);
    }
    volatile float t = (x - st[0]) * st[1];
    volatile float u = t * (1.0f + a->pv_buf[a->pv_off + kk]);
    return or_rf16(u + a->pv_buf[a->pv_off + a->pv_stride + kk]);
  }
  case P0K_X_CONV: {
    uint32_t Ci = a->c_Ci, tap = k / Ci, ci = k % Ci;
    uint32_t oy = row / a->c_Wo, ox = row % a->c_Wo;
    int iy = (int)(oy * c->stride + tap / c->ks) - (int)a->c_padT, ix = (int)(ox * c->stride + tap % c->ks) - (int)a->c_padL;
    int HH = a->c_up2 ? 2 * (int)a->c_Hi : (int)a->c_Hi, WW = a->c_up2 ? 2 * (int)a->c_Wi : (int)a->c_Wi;
    int ok = iy >= 0 && ix >= 0 && iy < HH && ix < WW;
    if (!ok) return 0.0f;
    uint32_t sy = (uint32_t)iy, sx = (uint32_t)ix;
    if (a->c_up2) { sy >>= 1; sx >>= 1; }
    if (sy > a->c_Hi - 1) sy = a->c_Hi - 1;
    if (sx > a->c_Wi - 1) sx = a->c_Wi - 1;
    float x = or_h2f(get16(xb + (((uint64_t)sy * a->c_Wi + sx) * Ci + ci) * 2));
    if (a->c_gn) {
      volatile float z = x * a->pv_buf[a->pv_off + ci] + a->pv_buf[a->pv_off + a->pv_stride + ci];
      return or_rf16(silu(z));
    }
    return x;
  }
  case P0K_X_CONV3: {
    uint32_t Ci = a->c_Ci, tap = k / Ci, ci = k % Ci, HW = a->c_Ho * a->c_Wo;
    uint32_t ot = row / HW, rem = row % HW, oy = rem / a->c_Wo, ox = rem % a->c_Wo;
    uint32_t kt = tap / 9, ky = (tap / 3) % 3, kx = tap % 3;
    int itg = (int)(ot + a->c_padT + kt) - 1;
    if (itg < 0) itg = 0;
    if (itg > (int)c->stride - 1) itg = (int)c->stride - 1;
    uint32_t it = c->ks > 1 ? (uint32_t)itg % c->ks : (uint32_t)itg - a->c_padL;
    int iy = (int)(oy + ky) - 1, ix = (int)(ox + kx) - 1;
    int ok = iy >= 0 && ix >= 0 && iy < (int)a->c_Hi && ix < (int)a->c_Wi;
    if (!ok) return 0.0f;
    uint64_t vox = ((uint64_t)it * a->c_Hi + (uint32_t)iy) * a->c_Wi + (uint32_t)ix;
    float x = or_h2f(get16(xb + (vox * Ci + ci) * 2));
    if (a->c_pn) {
      volatile float z = x * a->st_buf[vox];
      return or_rf16(silu(z));
    }
    return x;
  }
  }
  return 0.0f;
}

/* weight row of ws column n (gemm.js:98-101) */
static uint32_t wrow(const ocfg *c, uint32_t n) {
  const p0k_gemm_args *a = c->a;
  if (a->epi == P0K_EPI_SWIGLU) return ((n & 1u) ? a->wr1 : a->wr0) + (n >> 1);
  uint32_t r = a->wr0 + n;
  return r < c->Nw - 1 ? r : c->Nw - 1;
}

static uint16_t *y16(const ocfg *c, uint64_t i) { return (uint16_t *)((uint8_t *)c->a->y_buf + c->a->y_off) + i; }
static float *y32(const ocfg *c, uint64_t i) { return (float *)((uint8_t *)c->a->y_buf + c->a->y_off) + i; }

/* The argument struct this oracle reads, as include/p0k.h lays it out: its size and the byte offset of every field in
 * declaration order (the tests hold the oracle's own Python flattening of the reference's argument object to it). */
#define OR_OFF(f) off[n++] = (uint64_t)offsetof(p0k_gemm_args, f)
uint32_t or_gemm_args_layout(uint64_t *off, uint32_t cap) {
  uint32_t n = 0;
  if (cap < 80) return 0;
  off[n++] = sizeof(p0k_gemm_args);
  OR_OFF(struct_size); OR_OFF(w_enc); OR_OFF(w_buf); OR_OFF(w_off); OR_OFF(w_bytes); OR_OFF(w_rows); OR_OFF(w_cols);
  OR_OFF(w_ld); OR_OFF(x_buf); OR_OFF(x_off); OR_OFF(x_size); OR_OFF(x_ld); OR_OFF(x_k0); OR_OFF(x_mode); OR_OFF(y_buf);
  OR_OFF(y_off); OR_OFF(y_size); OR_OFF(y_ld); OR_OFF(y_n0); OR_OFF(M); OR_OFF(N); OR_OFF(K); OR_OFF(epi); OR_OFF(acc);
  OR_OFF(tile_bm); OR_OFF(tile_bn); OR_OFF(wr0); OR_OFF(wr1); OR_OFF(wk0); OR_OFF(ev_buf); OR_OFF(ev_off);
  OR_OFF(ev_size); OR_OFF(st_buf); OR_OFF(st_off); OR_OFF(st_size); OR_OFF(pv_buf); OR_OFF(pv_off); OR_OFF(pv_stride);
  OR_OFF(pv_size); OR_OFF(bv_buf); OR_OFF(bv_off); OR_OFF(bv_up); OR_OFF(bv_size); OR_OFF(gt_buf); OR_OFF(gt_size);
  OR_OFF(rope_buf); OR_OFF(rope_size); OR_OFF(res); OR_OFF(store); OR_OFF(act); OR_OFF(h_Ltot); OR_OFF(h_Hq);
  OR_OFF(h_Hkv); OR_OFF(h_rowOff); OR_OFF(h_eps); OR_OFF(h_rope_mode); OR_OFF(c_Hi); OR_OFF(c_Wi); OR_OFF(c_Ci);
  OR_OFF(c_Ho); OR_OFF(c_Wo); OR_OFF(c_stride); OR_OFF(c_padT); OR_OFF(c_padL); OR_OFF(c_ks); OR_OFF(c_up2);
  OR_OFF(c_gn); OR_OFF(c_pn);
  return n;
}
#undef OR_OFF

int or_gemm(const p0k_gemm_args *a, uint32_t m0, uint32_t m1) {
  if (!a || !a->x_buf || !a->w_buf || !a->y_buf || a->K % 32) return -1;
  ocfg c = { a, a->x_ld ? a->x_ld : a->K, a->y_ld ? a->y_ld : a->N, 0, a->w_rows, a->c_ks ? a->c_ks : 1,
             a->c_stride ? a->c_stride : 1, 0, a->h_eps != 0.0f ? a->h_eps : 1e-6f };
  c.wG = a->w_enc == P0K_ENC_Q4G32A_T64 ? a->w_cols / 32 : a->w_enc == P0K_ENC_Q8G64S_T64 ? a->w_cols / 64
         : (a->w_ld ? a->w_ld : a->w_cols);
  const uint8_t *wb = (const uint8_t *)a->w_buf + a->w_off;
  uint32_t N = a->N, K = a->K;
  if (m1 > a->M) m1 = a->M;
  float *xr = (float *)malloc(sizeof(float) * K);
  double *acc = (double *)malloc(sizeof(double) * (N ? N : 1));
  float *wcol = (float *)malloc(sizeof(float) * K);
  /* the weights are decoded once per call into fp32 rows (fp16 values) */
  float *Wd = (float *)malloc(sizeof(float) * (uint64_t)N * K);
  for (uint32_t n = 0; n < N; n++) {
    uint32_t r = wrow(&c, n);
    for (uint32_t k = 0; k < K; k++) Wd[(uint64_t)n * K + k] = weight_value(a->w_enc, wb, c.wG, r, a->wk0 + k);
  }
  (void)wcol;
  for (uint32_t m = m0; m < m1; m++) {
    for (uint32_t k = 0; k < K; k++) xr[k] = xprime(&c, m, k);
    for (uint32_t n = 0; n < N; n++) {
      double s = 0.0; const float *w = Wd + (uint64_t)n * K;
      for (uint32_t k = 0; k < K; k++) s += (double)xr[k] * (double)w[k];
      acc[n] = s;
    }
    uint64_t yrow = (uint64_t)m * c.ldy + a->y_n0;
    switch (a->epi) {
    case P0K_EPI_F16:                                                        /* gemm.js:194-196 */
      for (uint32_t n = 0; n < N; n++) *y16(&c, yrow + n) = or_f2h((float)acc[n]);
      break;
    case P0K_EPI_F32:
      for (uint32_t n = 0; n < N; n++) *y32(&c, yrow + n) = (float)acc[n];
      break;
    case P0K_EPI_RESADD:                                                     /* gemm.js:197-203 */
      for (uint32_t n = 0; n < N; n++) {
        double g = a->ev_buf ? a->ev_buf[a->ev_off + n] : 1.0, b = a->bv_buf ? a->bv_buf[a->bv_off + n] : 0.0;
        double prev = a->store ? 0.0 : *y32(&c, yrow + n);
        *y32(&c, yrow + n) = (float)(prev + g * (acc[n] + b));
      }
      break;
    case P0K_EPI_BIAS:                                                       /* gemm.js:211-215 */
      for (uint32_t n = 0; n < N; n++) {
        double v = acc[n] + a->ev_buf[a->ev_off + n];
        if (a->res) v += or_h2f(*y16(&c, yrow + n));
        *y16(&c, yrow + n) = or_f2h((float)v);
      }
      break;
    case P0K_EPI_SWIGLU:                                                     /* gemm.js:204-210 */
      for (uint32_t o = 0; o < N / 2; o++) {
        double g = acc[2 * o], u = acc[2 * o + 1];
        if (a->bv_buf) { g += a->bv_buf[a->bv_off + o]; u += a->bv_buf[a->bv_off + a->bv_up + o]; }
        double act;
        if (a->act == P0K_ACT_GELU) {
          double t = 0.7978845608 * (g + 0.044715 * g * g * g);
          if (t > 15) t = 15;
          if (t < -15) t = -15;
          act = g * 0.5 * (1.0 + tanh(t));
        } else act = g / (1.0 + exp(-g));
        *y16(&c, yrow + o) = or_f2h((float)(act * u));
      }
      break;
    case P0K_EPI_HEADS: {                                                    /* gemm.js:216-253 */
      uint32_t row = a->h_rowOff + m;
      for (uint32_t hd = 0; hd < N / 128; hd++) {
        double v[128];
        for (int d = 0; d < 128; d++) v[d] = acc[hd * 128 + d];
        int sec = hd < a->h_Hq ? 0 : hd < a->h_Hq + a->h_Hkv ? 1 : 2;
        if (sec < 2) {
          double ss = 0; for (int d = 0; d < 128; d++) ss += v[d] * v[d];
          double inv = 1.0 / sqrt(ss / 128.0 + c.eps);
          const float *nw = a->ev_buf + a->ev_off + (sec ? 128 : 0);
          for (int d = 0; d < 128; d++) v[d] = v[d] * inv * nw[d];
          const float *rp = a->rope_buf + (uint64_t)row * 128;
          if (a->h_rope_mode == P0K_ROPE_HALF) {                             /* pair (d, d + 64), angle d */
            for (int d = 0; d < 64; d++) {
              double cs = rp[2 * d], sn = rp[2 * d + 1], lo = v[d], hi = v[d + 64];
              v[d] = lo * cs - hi * sn; v[d + 64] = hi * cs + lo * sn;
            }
          } else {                                                           /* pair (2p, 2p + 1), angle p */
            for (int p = 0; p < 64; p++) {
              double cs = rp[2 * p], sn = rp[2 * p + 1], x0 = v[2 * p], x1 = v[2 * p + 1];
              v[2 * p] = x0 * cs - x1 * sn; v[2 * p + 1] = x0 * sn + x1 * cs;
            }
          }
        }
        uint64_t ob = ((uint64_t)hd * a->h_Ltot + row) * 128;
        for (int d = 0; d < 128; d++) *y16(&c, ob + d) = or_f2h((float)v[d]);
      }
      break;
    }
    case P0K_EPI_ONORMGATE: {                                                /* gemm.js:227-232 */
      const uint16_t *gt = (const uint16_t *)a->gt_buf;
      for (uint32_t nb = 0; nb < N; nb += 128) {
        double ss = 0; for (int d = 0; d < 128; d++) ss += acc[nb + d] * acc[nb + d];
        double inv = 1.0 / sqrt(ss / 128.0 + c.eps);
        for (int d = 0; d < 128; d++) {
          double g = or_h2f(gt[(uint64_t)m * a->h_Ltot + a->y_n0 + nb + d]);
          double v = acc[nb + d] * inv * a->ev_buf[a->ev_off + d] / (1.0 + exp(-g));
          *y16(&c, yrow + nb + d) = or_f2h((float)v);
        }
      }
      break;
    }
    default: break;
    }
  }
  free(Wd); free(wcol); free(acc); free(xr);
  return 0;
}

/* ------------------------------------------------------------------ row statistics (src/ops/misc.js:16-44) */
int or_rowstats(const p0k_rowstats_args *a) {
  uint32_t ld = a->ld ? a->ld : a->cols;
  const float *x = (const float *)((const uint8_t *)a->x_buf + a->x_off);
  for (uint32_t r = 0; r < a->rows; r++) {
    const float *row = x + (uint64_t)r * ld + a->c0;
    double mean = 0;
    if (a->mode == 0) { for (uint32_t i = 0; i < a->cols; i++) mean += row[i]; mean /= a->cols; }
    double q = 0;
    for (uint32_t i = 0; i < a->cols; i++) { double d = row[i] - mean; q += d * d; }
    double var = q / a->cols;
    a->st_buf[(uint64_t)(a->st_off + r) * 2] = (float)mean;
    a->st_buf[(uint64_t)(a->st_off + r) * 2 + 1] = (float)(1.0 / sqrt(var + a->eps));
  }
  return 0;
}

/* ------------------------------------------------------------------ the test suite's references */
void or_cpu_gemm(const float *X, const float *W, int M, int N, int K, float *Y) {      /* test/kernels.test.js:29 */
  for (int m = 0; m < M; m++)
    for (int n = 0; n < N; n++) {
      double s = 0;
      for (int k = 0; k < K; k++) s += (double)X[(int64_t)m * K + k] * W[(int64_t)n * K + k];
      Y[(int64_t)m * N + n] = (float)s;
    }
}

void or_cpu_conv3(const float *X, const float *Wt, int T, int H, int W, int C, int N, float *Y) {   /* :52-65 */
  int K = 27 * C;
  for (int t = 0; t < T; t++)
    for (int y = 0; y < H; y++)
      for (int x = 0; x < W; x++)
        for (int n = 0; n < N; n++) {
          double s = 0;
          for (int kt = 0; kt < 3; kt++)
            for (int ky = 0; ky < 3; ky++)
              for (int kx = 0; kx < 3; kx++) {
                int it = t + kt - 1, iy = y + ky - 1, ix = x + kx - 1;
                if (it < 0) it = 0;
                if (it > T - 1) it = T - 1;
                if (iy < 0 || ix < 0 || iy >= H || ix >= W) continue;
                const float *xp = X + (((int64_t)it * H + iy) * W + ix) * C;
                const float *wp = Wt + (int64_t)n * K + (kt * 9 + ky * 3 + kx) * C;
                for (int c = 0; c < C; c++) s += (double)xp[c] * wp[c];
              }
          Y[(((int64_t)t * H + y) * W + x) * N + n] = (float)s;
        }
}

/* ------------------------------------------------------------------ pixstats / GroupNorm statistics */
void or_pixstats(const uint16_t *x, uint32_t V, uint32_t C, float eps, float *r) {
  for (uint32_t v = 0; v < V; v++) {
    double s = 0;
    for (uint32_t c = 0; c < C; c++) { double t = or_h2f(x[(uint64_t)v * C + c]); s += t * t; }
    r[v] = (float)(1.0 / sqrt(s / C + (double)eps));
  }
}

void or_gn_partial(const uint16_t *x, uint32_t pix, uint32_t C, float *part) {
  const uint32_t cpg = C / 32, nwg = (pix + 63) / 64;
  for (uint32_t w = 0; w < nwg; w++) {
    const uint32_t p0 = w * 64, np = pix - p0 < 64 ? pix - p0 : 64;
    for (uint32_t g = 0; g < 32; g++) {
      double s = 0, m2 = 0, n = (double)np * cpg;
      for (uint32_t p = p0; p < p0 + np; p++)
        for (uint32_t c = g * cpg; c < (g + 1) * cpg; c++) s += or_h2f(x[(uint64_t)p * C + c]);
      double mean = s / (n > 1 ? n : 1);
      for (uint32_t p = p0; p < p0 + np; p++)
        for (uint32_t c = g * cpg; c < (g + 1) * cpg; c++) { double d = or_h2f(x[(uint64_t)p * C + c]) - mean; m2 += d * d; }
      float *q = part + ((uint64_t)w * 32 + g) * 4;
      q[0] = (float)n; q[1] = (float)mean; q[2] = (float)m2; q[3] = 0.0f;
    }
  }
}

void or_gn_finalize(const float *part, uint32_t nwg, uint32_t C, float eps, const float *gamma, const float *beta,
                    float *ab) {
  const uint32_t cpg = C / 32;
  for (uint32_t g = 0; g < 32; g++) {
    double n = 0, mean = 0, m2 = 0;
    for (uint32_t w = 0; w < nwg; w++) {
      const float *q = part + ((uint64_t)w * 32 + g) * 4;
      if (q[0] > 0) {
        double nn = n + q[0], d = q[1] - mean;
        mean += d * (q[0] / nn);
        m2 += q[2] + d * d * (n * q[0] / nn);
        n = nn;
      }
    }
    double rs = 1.0 / sqrt(m2 / (n > 1 ? n : 1) + (double)eps);
    for (uint32_t c = g * cpg; c < (g + 1) * cpg; c++) {
      double a = gamma[c] * rs;
      ab[c] = (float)a;
      ab[C + c] = (float)(beta[c] - mean * a);
    }
  }
}

/* ------------------------------------------------------------------ attention (cpuAttn, test/kernels.test.js:30-49) */
void or_attention(const uint16_t *Q, const uint16_t *K, const uint16_t *V, uint16_t *O, uint32_t Lq, uint32_t Lk,
                  uint32_t Hq, uint32_t Hkv, uint32_t ldo, uint32_t mode, uint32_t nvalid, float scale, float cap) {
  const uint32_t D = 128, grp = Hq / Hkv;
  double *s = (double *)malloc(sizeof(double) * (Lk ? Lk : 1));
  for (uint32_t h = 0; h < Hq; h++) {
    const uint32_t kh = h / grp;
    for (uint32_t i = 0; i < Lq; i++) {
      double mx = -INFINITY;
      for (uint32_t j = 0; j < Lk; j++) {
        int vis = mode == 1 ? j <= (i < nvalid - 1 ? i : nvalid - 1) : mode == 2 ? j < nvalid : 1;
        if (!vis) { s[j] = -INFINITY; continue; }
        double a = 0;
        for (uint32_t d = 0; d < D; d++)
          a += (double)or_h2f(Q[((uint64_t)h * Lq + i) * D + d]) * or_h2f(K[((uint64_t)kh * Lk + j) * D + d]);
        a *= scale;
        if (cap > 0) a = cap * tanh(a / cap);
        s[j] = a;
        if (a > mx) mx = a;
      }
      double sum = 0;
      for (uint32_t j = 0; j < Lk; j++) { s[j] = s[j] == -INFINITY ? 0 : exp(s[j] - mx); sum += s[j]; }
      for (uint32_t d = 0; d < D; d++) {
        double a = 0;
        for (uint32_t j = 0; j < Lk; j++) if (s[j] != 0) a += s[j] * or_h2f(V[((uint64_t)kh * Lk + j) * D + d]);
        O[(uint64_t)i * ldo + h * D + d] = or_f2h((float)(a / sum));
      }
    }
  }
  free(s);
}
