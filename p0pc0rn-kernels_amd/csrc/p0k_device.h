// p0k_device.h — device-side pieces shared by the GEMM (MFMA) and GEMV kernels of the `gemm` op, gfx950 only.
//
//  * Params: the kernel argument block. It carries the same fields as the reference's uniform P (src/ops/gemm.js:39-41)
//    plus the operand pointers (X, W, Y already advanced by their byte offsets).
//  * Weight decoding from the FORMAT.md records straight into packed fp16 pairs (v_perm / v_and_or + v_pk_fma_f16).
//  * The prologue: X' = f16(prologue(X)) for 8 consecutive k of one row (gemm.js:60-95).
//  * The epilogue over an fp32 tile of 128 ws columns held in LDS (gemm.js:191-254).
//
// K order inside an 8-k block. The decoders emit fp16 PAIRS in the order that costs the fewest instructions:
//   q4 (one u32 word = 8 codes, nibble i = k i):   pairs (0,4) (1,5) (2,6) (3,7)
//   q8 (one u32 word = 4 codes, byte i = k i):     pairs (0,2) (1,3)
//   f16:                                           pairs (0,1) (2,3) (4,5) (6,7)
// X' is stored in the same order (xperm()), so a dot product over the block sees matching k on both sides; a sum over
// k does not depend on the order the terms are paired in. The decoded VALUES are bit-exact with the reference's
// f16(q*s + mn) / f16(q*s) (gemm.js:152,163); see dq_q4_word.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace p0k {

typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

enum { W_Q4 = 1, W_Q8 = 2, W_F16 = 3 };
enum { X_F16 = 0, X_LNMOD = 1, X_RMS = 2, X_CONV = 3, X_CONV3 = 4 };
enum { E_F16 = 0, E_F32 = 1, E_RESADD = 2, E_SWIGLU = 3, E_HEADS = 4, E_BIAS = 5, E_ONORMGATE = 6 };
enum {
  F_GATE = 1, F_BIAS = 2, F_STORE = 4, F_RES = 8, F_GELU = 16, F_ROPE_HALF = 32, F_PN = 64, F_GN = 128, F_UP2 = 256,
  F_XALIGN8 = 512,   // X rows / k0 allow 16-byte loads of 8 halfs (else two 8-byte loads)
  F_WALIGN8 = 1024,  // f16 weight rows / k0 allow 16-byte loads
};

struct Params {
  const uint8_t *W;   // weight tensor (w.buf + w.off)
  const uint8_t *X;   // activations   (x.buf + x.off)
  uint8_t *Y;         // output        (y.buf + y.off)
  const float *ST, *PV, *EV, *BV, *RP;
  const uint16_t *GT;
  uint32_t M, N, K, ldx, kx0, wR0, wR1, wG, wk0, ldy, ny0;
  uint32_t rowOff, Ltot, Hq, Hkv;
  float eps;
  uint32_t pvOff, pvStride, evOff, statOff;
  uint32_t Hi, Wi, Ci, Ho, Wo, stride, padT, padL, ks, Nw, bvOff, bvUp;
  uint32_t flags;
  int32_t epi;
  uint32_t tilesM, tilesN;
  const uint8_t *Z;    // 16 zero bytes (the load-to-LDS conv3 gather reads them for padding taps)
  uint32_t nvox;       // conv3: input voxels the call may read (frames x Hi x Wi)
  uint32_t nbase;      // load-to-LDS GEMM: first ws column of this launch (its tiles cover [nbase, N))
};

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) { return __builtin_amdgcn_perm(hi, lo, sel); }

// Streaming reads of data used once per call (the decode's weights): buffer loads at 32-bit byte offsets from a raw
// buffer resource over the tensor, cache policy "sc0 nt" (non-temporal). They move the decode's 73 MB about 1.5 %
// faster than global loads with the nt bit alone.
typedef __amdgpu_buffer_rsrc_t srsrc;
__device__ __forceinline__ srsrc stream_rsrc(const uint8_t *base) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)0xffffffff, 0x00020000);
}
constexpr int SC0_NT = 3;   // buffer-load cache policy bits on gfx950: 1 = sc0, 2 = nt
__device__ __forceinline__ u32x4 sload128(srsrc r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, SC0_NT));
}
__device__ __forceinline__ u32x2 sload64(srsrc r, uint32_t off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, SC0_NT));
}
__device__ __forceinline__ uint32_t sload32(srsrc r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, SC0_NT); }
// System-coherent 16-byte vector accesses (cache policy sc0 sc1: they skip the per-XCD L2s, so workgroups on different
// XCDs exchange data through memory without any L2 writeback or invalidation; a store counts as done only once it is
// there): the split-K partials of the decode.
constexpr int SC0_SC1 = 17;
__device__ __forceinline__ void sys_store128(srsrc r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)off, 0, SC0_SC1);
}
__device__ __forceinline__ u32x4 sys_load128(srsrc r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, SC0_SC1));
}
__device__ __forceinline__ f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
__device__ __forceinline__ uint32_t as_u(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }

// ----------------------------------------------------------------------------------------------- weight rows
// ws column n -> weight row (gemm.js:98-101). GLU columns interleave (gate, up); rows are clamped to the tensor for
// LOADS only (columns past N are never stored), which keeps every read inside the weight buffer.
__device__ __forceinline__ uint32_t wrow(const Params &p, uint32_t n) {
  uint32_t r = (p.epi == E_SWIGLU) ? (((n & 1u) ? p.wR1 : p.wR0) + (n >> 1)) : (p.wR0 + n);
  return r < p.Nw - 1u ? r : p.Nw - 1u;
}

// ----------------------------------------------------------------------------------------------- decoders
// q4g32a.t64: one code word (k = 8w..8w+7 of the group) + its (scale, min) word -> 4 fp16 pairs (0,4)(1,5)(2,6)(3,7).
// Fast path: (0x6400 | q) is the fp16 1024 + q; minus 1024 gives q exactly; v_pk_fma_f16 then rounds q*s + mn once.
// The reference rounds q*s + mn to fp32 first and then to fp16 (gemm.js:151-152). Both agree whenever q*s + mn is
// exact in fp32: q*s has at most 15 significant bits, mn 11, so the sum fits fp32's 24 bits when the exponents satisfy
// -8 <= E(mn) - E(s) <= 12 (or mn = 0). Other (scale, min) words take the fp32 path, which is the reference's formula.
__device__ __forceinline__ bool q4_fast_ok(uint32_t sm) {
  // branch-free (it sits inside unrolled streaming loops): exponent fields, 0 counted as 1 (subnormals)
  const uint32_t mb = sm >> 16;
  const int es = (int)((sm >> 10) & 31u), em = (int)((mb >> 10) & 31u);
  const int d = (em | (em == 0)) - (es | (es == 0));
  const bool finite = (es != 31) & (em != 31);
  return finite & (((mb & 0x7fffu) == 0u) | ((d >= -8) & (d <= 12)));
}
__device__ __forceinline__ void dq_q4_word(uint32_t w, uint32_t sm, bool fast, f16x2 out[4]) {
  if (fast) {
    f16x2 s2 = as_h2(perm(sm, sm, 0x01000100u)), m2 = as_h2(perm(sm, sm, 0x03020302u));
    const f16x2 k1024 = {(f16)1024.0f, (f16)1024.0f};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      uint32_t v = ((w >> (4 * i)) & 0x000F000Fu) | 0x64006400u;
      out[i] = __builtin_elementwise_fma(as_h2(v) - k1024, s2, m2);
    }
  } else {
    f16x2 sm2 = as_h2(sm);
    float s = (float)sm2.x, mn = (float)sm2.y;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float a = fmaf((float)((w >> (4 * i)) & 15u), s, mn), b = fmaf((float)((w >> (4 * i + 16)) & 15u), s, mn);
      // keep the fp32 rounding: without the barrier the compiler fuses fma + cvt into v_fma_mix (one rounding)
      asm volatile("" : "+v"(a), "+v"(b));
      out[i] = (f16x2){(f16)a, (f16)b};
    }
  }
}
// q8g64s.t64: one code word (4 int8, k = 4w..4w+3) -> 2 fp16 pairs (0,2)(1,3). (b ^ 0x80) | 0x6400 is the fp16
// 1024 + b + 128; minus 1152 gives the signed code exactly, and q*s (19 significant bits at most) is rounded once,
// as f16(q*s) in the reference (gemm.js:162-163).
__device__ __forceinline__ void dq_q8_word(uint32_t w, f16x2 s2, f16x2 out[2]) {
  uint32_t u = w ^ 0x80808080u;
  const f16x2 k1152 = {(f16)1152.0f, (f16)1152.0f};
  out[0] = (as_h2(perm(0x64646464u, u, 0x04020400u)) - k1152) * s2;
  out[1] = (as_h2(perm(0x64646464u, u, 0x04030401u)) - k1152) * s2;
}

// X' block of 8 halfs (natural order, 4 u32) -> the pair order of the weight encoding
template <int WE>
__device__ __forceinline__ u32x4 xperm(u32x4 v) {
  if constexpr (WE == W_Q4) {
    return (u32x4){perm(v.z, v.x, 0x05040100u), perm(v.z, v.x, 0x07060302u), perm(v.w, v.y, 0x05040100u),
                   perm(v.w, v.y, 0x07060302u)};
  } else if constexpr (WE == W_Q8) {
    return (u32x4){perm(v.y, v.x, 0x05040100u), perm(v.y, v.x, 0x07060302u), perm(v.w, v.z, 0x05040100u),
                   perm(v.w, v.z, 0x07060302u)};
  } else {
    return v;
  }
}

__device__ __forceinline__ uint32_t pack2(float a, float b) { return as_u((f16x2){(f16)a, (f16)b}); }
// e^x as 2^(x log2 e) on the hardware exp2 (v_exp_f32) and 1 / x on the hardware reciprocal (v_rcp_f32), each
// within about one fp32 ulp, far inside the fp16 rounding of every result they feed; the logistic function
// 1 / (1 + e^-x) from them saturates cleanly (e^-x = inf -> 0)
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float sigmoid(float x) { return __builtin_amdgcn_rcpf(1.0f + fast_exp(-x)); }
__device__ __forceinline__ float silu(float z) { return z * sigmoid(z); }

// ----------------------------------------------------------------------------------------------- prologue
// Row context of the implicit-GEMM convolutions: computed once per row, reused for every k step.
struct RowCtx {
  int a, b, c;   // conv3: (ot, oy, ox); conv: (oy, ox, -)
};
template <int XM>
__device__ __forceinline__ RowCtx row_ctx(const Params &p, uint32_t row) {
  RowCtx r{0, 0, 0};
  if constexpr (XM == X_CONV3) {
    uint32_t HW = p.Ho * p.Wo, ot = row / HW, rem = row - ot * HW, oy = rem / p.Wo;
    r.a = (int)ot; r.b = (int)oy; r.c = (int)(rem - oy * p.Wo);
  } else if constexpr (XM == X_CONV) {
    uint32_t oy = row / p.Wo;
    r.a = (int)oy; r.b = (int)(row - oy * p.Wo);
  }
  return r;
}

// X' for k = k .. k+7 of row `row` (row < M), as 4 packed fp16 pairs in NATURAL order. (gemm.js:60-95)
// For conv / conv3, the 8 k lie inside one tap because Ci % 32 == 0 (checked on the host).
// XA: f16 rows are 16-byte aligned (1), not (0), or as F_XALIGN8 says (2; a branch per load).
template <int XM, int XA = 2>
__device__ __forceinline__ u32x4 xload8(const Params &p, uint32_t row, const RowCtx &rc, uint32_t k) {
  if constexpr (XM == X_F16) {
    const uint8_t *src = p.X + ((size_t)row * p.ldx + p.kx0 + k) * 2;
    if (XA == 1 || (XA == 2 && (p.flags & F_XALIGN8))) return *(const u32x4 *)src;
    u32x2 lo = *(const u32x2 *)src, hi = *(const u32x2 *)(src + 8);
    return (u32x4){lo.x, lo.y, hi.x, hi.y};
  } else if constexpr (XM == X_RMS || XM == X_LNMOD) {
#pragma clang fp contract(off)   // one fp32 rounding per operation, in the reference's order, before the fp16 rounding
    const f32x4 *src = (const f32x4 *)(p.X + ((size_t)row * p.ldx + p.kx0 + k) * 4);
    f32x4 x0 = src[0], x1 = src[1];
    const float *st = p.ST + (size_t)(p.statOff + row) * 2;
    float mean = st[0], rstd = st[1];
    const f32x4 *g = (const f32x4 *)(p.PV + p.pvOff + p.kx0 + k);
    f32x4 g0 = g[0], g1 = g[1], y0, y1;
    if constexpr (XM == X_RMS) {                       // X' = x * rstd * w[k]
      y0 = x0 * rstd * g0; y1 = x1 * rstd * g1;
    } else {                                           // X' = (x - mean) * rstd * (1 + scale[k]) + shift[k]
      const f32x4 *h = (const f32x4 *)(p.PV + p.pvOff + p.pvStride + p.kx0 + k);
      f32x4 h0 = h[0], h1 = h[1];
      y0 = (x0 - mean) * rstd * (1.0f + g0) + h0; y1 = (x1 - mean) * rstd * (1.0f + g1) + h1;
    }
    return (u32x4){pack2(y0.x, y0.y), pack2(y0.z, y0.w), pack2(y1.x, y1.y), pack2(y1.z, y1.w)};
  } else if constexpr (XM == X_CONV3) {
    uint32_t tap = k / p.Ci, c0 = k - tap * p.Ci, kt = tap / 9u, r9 = tap - kt * 9u, ky = r9 / 3u, kx = r9 - ky * 3u;
    int itg = rc.a + (int)(p.padT + kt) - 1;
    itg = itg < 0 ? 0 : (itg > (int)p.stride - 1 ? (int)p.stride - 1 : itg);
    uint32_t it = p.ks > 1u ? (uint32_t)itg % p.ks : (uint32_t)itg - p.padL;
    int iy = rc.b + (int)ky - 1, ix = rc.c + (int)kx - 1;
    if (iy < 0 || ix < 0 || iy >= (int)p.Hi || ix >= (int)p.Wi) return (u32x4){0u, 0u, 0u, 0u};
    size_t vox = ((size_t)it * p.Hi + (uint32_t)iy) * p.Wi + (uint32_t)ix;
    u32x4 v = *(const u32x4 *)(p.X + (vox * p.Ci + c0) * 2);
    if (p.flags & F_PN) {                              // PixelNorm + SiLU before the zero padding (gemm.js:77-79)
      float sc = p.ST[vox];
      f16x2 a = as_h2(v.x), b = as_h2(v.y), c = as_h2(v.z), d = as_h2(v.w);
      v = (u32x4){pack2(silu((float)a.x * sc), silu((float)a.y * sc)), pack2(silu((float)b.x * sc), silu((float)b.y * sc)),
                  pack2(silu((float)c.x * sc), silu((float)c.y * sc)), pack2(silu((float)d.x * sc), silu((float)d.y * sc))};
    }
    return v;
  } else {   // X_CONV, 2-D over HWC (gemm.js:81-91)
    uint32_t tap = k / p.Ci, c0 = k - tap * p.Ci;
    int iy = rc.a * (int)p.stride + (int)(tap / p.ks) - (int)p.padT;
    int ix = rc.b * (int)p.stride + (int)(tap % p.ks) - (int)p.padL;
    bool up2 = p.flags & F_UP2;
    int HH = up2 ? 2 * (int)p.Hi : (int)p.Hi, WW = up2 ? 2 * (int)p.Wi : (int)p.Wi;
    if (iy < 0 || ix < 0 || iy >= HH || ix >= WW) return (u32x4){0u, 0u, 0u, 0u};
    uint32_t sy = up2 ? ((uint32_t)iy >> 1) : (uint32_t)iy, sx = up2 ? ((uint32_t)ix >> 1) : (uint32_t)ix;
    sy = sy < p.Hi - 1u ? sy : p.Hi - 1u; sx = sx < p.Wi - 1u ? sx : p.Wi - 1u;
    u32x4 v = *(const u32x4 *)(p.X + (((size_t)sy * p.Wi + sx) * p.Ci + c0) * 2);
    if (p.flags & F_GN) {                              // GroupNorm-apply + SiLU before the zero padding
      const float *ga = p.PV + p.pvOff + c0, *gb = p.PV + p.pvOff + p.pvStride + c0;
      f16x2 h[4] = {as_h2(v.x), as_h2(v.y), as_h2(v.z), as_h2(v.w)};
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; i++)
        o[i] = pack2(silu((float)h[i].x * ga[2 * i] + gb[2 * i]), silu((float)h[i].y * ga[2 * i + 1] + gb[2 * i + 1]));
      v = (u32x4){o[0], o[1], o[2], o[3]};
    }
    return v;
  }
}

// ----------------------------------------------------------------------------------------------- epilogue
__device__ __forceinline__ uint16_t h_bits(float v) { return __builtin_bit_cast(uint16_t, (f16)v); }
__device__ __forceinline__ float h_val(uint16_t b) { return (float)__builtin_bit_cast(f16, b); }

__device__ __forceinline__ void store_f16x8(uint8_t *yb, size_t idx, const float v[8], uint32_t nvalid) {
  uint16_t *y = (uint16_t *)yb + idx;
  if (nvalid >= 8 && (((uintptr_t)y) & 15u) == 0) {
    *(u32x4 *)y = (u32x4){pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7])};
  } else {
    for (uint32_t j = 0; j < 8 && j < nvalid; j++) y[j] = h_bits(v[j]);
  }
}

// the GLU activation of gemm.js:205-209: SiLU g / (1 + e^-g), or tanh-GELU g (1 + tanh z) / 2 with its argument z
// clamped to +-15, computed as g * sigmoid(2 z) (the same function: (1 + tanh z) / 2 = 1 / (1 + e^-2z))
__device__ __forceinline__ float glu_act(float gt, bool gelu) {
  if (gelu) {
    float z = 0.7978845608f * (gt + 0.044715f * gt * gt * gt);
    z = fminf(fmaxf(z, -15.0f), 15.0f);
    return gt * sigmoid(2.0f * z);
  }
  return silu(gt);
}

// sum over the 16 lanes of an aligned lane group (the 16 threads that share one row in the epilogue)
__device__ __forceinline__ float sum16(float v) {
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) v += __shfl_xor(v, o, 16);
  return v;
}

// Apply the epilogue to rows [0, R) x 128 ws columns of an fp32 tile C (row stride ldc) whose first row is output row
// mB and first ws column is nB. Every thread of the block calls it (NT threads, NT % 16 == 0). Sixteen consecutive
// threads share one row, each owning 8 consecutive columns, so stores are 16 bytes and row reductions are shuffles.
template <int NT>
__device__ void epilogue(const Params &p, const float *C, int ldc, int R, uint32_t mB, uint32_t nB, int tid) {
  const int epi = p.epi;
  const int g = tid & 15;                       // 8-column group of the row
  constexpr int RPP = NT / 16;                  // rows per pass
  if (epi == E_SWIGLU) {                                                           // gemm.js:204-210
    // 8 output columns (16 ws columns, interleaved gate / up) per thread, 8 threads per row
    const uint32_t Nout = p.N >> 1;
    const bool bias = p.flags & F_BIAS, gelu = p.flags & F_GELU;
    for (int t = tid; t < R * 8; t += NT) {
      int r = t >> 3, ch = t & 7;
      uint32_t m = mB + r, o = (nB >> 1) + ch * 8;
      if (m >= p.M || o >= Nout) continue;
      const float *src = C + r * ldc + ch * 16;
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        float gt = src[2 * j], u = src[2 * j + 1];
        if (bias && o + j < Nout) { gt += p.BV[p.bvOff + o + j]; u += p.BV[p.bvOff + p.bvUp + o + j]; }
        v[j] = glu_act(gt, gelu) * u;
      }
      store_f16x8(p.Y, (size_t)m * p.ldy + p.ny0 + o, v, Nout - o);
    }
    return;
  }
  if (epi == E_HEADS) {                                                            // gemm.js:216-253
    // Q / K heads: RMSNorm over the head's 128 columns, the section's norm weights (loaded once here), RoPE from the
    // table row of each output row (prefetched one pass ahead, so only the first pass waits for its loads); V raw
    // a tile reaching past N covers heads that do not exist (N is a multiple of 128): nothing to write for them
    if (nB >= p.N) return;
    const uint32_t hd = nB >> 7;
    const int sec = hd < p.Hq ? 0 : (hd < p.Hq + p.Hkv ? 1 : 2);
    const int d0 = g * 8;
    const bool half = p.flags & F_ROPE_HALF;
    float nw[8];
    if (sec < 2) {
      const float *np = p.EV + p.evOff + (sec ? 128 : 0) + d0;   // ev.off is any float offset: scalar loads
#pragma unroll
      for (int j = 0; j < 8; j++) nw[j] = np[j];
    }
    // the (cos, sin) values a thread reads for one row: interleaved, pairs d0 / 2 .. + 3 (8 floats at d0);
    // rotate-half, angles (d0 + j) & 63, j = 0..7 (16 floats at 2 ((d0 & 63))); the table starts its buffer and a row
    // is 512 bytes, so these are 16-byte aligned
    auto rope_load = [&](int r0, f32x4 *dst) __attribute__((always_inline)) {
      const int r = r0 + (tid >> 4);
      const uint32_t m = mB + r, row = p.rowOff + (r < R && m < p.M ? m : 0u);
      const f32x4 *rp4 = (const f32x4 *)(p.RP + (size_t)row * 128 + (half ? 2 * (d0 & 63) : d0));
      dst[0] = rp4[0]; dst[1] = rp4[1];
      if (half) { dst[2] = rp4[2]; dst[3] = rp4[3]; }
    };
    f32x4 rc[4], rn[4];
    if (sec < 2) rope_load(0, rc);
    for (int r0 = 0; r0 < R; r0 += RPP) {
      const int r = r0 + (tid >> 4);
      const uint32_t m = mB + r;
      const bool live = r < R && m < p.M;          // whole 16-lane groups agree, so the shuffles below are safe
      if (sec < 2 && r0 + RPP < R) rope_load(r0 + RPP, rn);
      float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      if (r < R) {
        const f32x4 *src = (const f32x4 *)(C + r * ldc + g * 8);
        f32x4 a0 = src[0], a1 = src[1];
        v[0] = a0.x; v[1] = a0.y; v[2] = a0.z; v[3] = a0.w; v[4] = a1.x; v[5] = a1.y; v[6] = a1.z; v[7] = a1.w;
      }
      if (sec < 2) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) ss += v[j] * v[j];
        ss = sum16(ss);
        const float inv = __frsqrt_rn(ss / 128.0f + p.eps);
        float x[8];
#pragma unroll
        for (int j = 0; j < 8; j++) x[j] = v[j] * inv * nw[j];
        const float rp[16] = {rc[0].x, rc[0].y, rc[0].z, rc[0].w, rc[1].x, rc[1].y, rc[1].z, rc[1].w,
                              rc[2].x, rc[2].y, rc[2].z, rc[2].w, rc[3].x, rc[3].y, rc[3].z, rc[3].w};
        if (!half) {                             // interleaved pairs (2p, 2p+1), angle p
#pragma unroll
          for (int j = 0; j < 8; j += 2) {
            const float cs = rp[j], sn = rp[j + 1];
            v[j] = x[j] * cs - x[j + 1] * sn;
            v[j + 1] = x[j] * sn + x[j + 1] * cs;
          }
        } else {                                 // rotate-half pairs (d, d+64): the partner columns are 8 groups away
          float y[8];
#pragma unroll
          for (int j = 0; j < 8; j++) y[j] = __shfl_xor(x[j], 8, 16);
          const bool lo = d0 < 64;
#pragma unroll
          for (int j = 0; j < 8; j++) {
            const float cs = rp[2 * j], sn = rp[2 * j + 1];
            v[j] = lo ? x[j] * cs - y[j] * sn : x[j] * cs + y[j] * sn;
          }
        }
#pragma unroll
        for (int q = 0; q < 4; q++) rc[q] = rn[q];
      }
      if (live) store_f16x8(p.Y, ((size_t)hd * p.Ltot + p.rowOff + m) * 128 + d0, v, 8);
    }
    return;
  }
  for (int r0 = 0; r0 < R; r0 += RPP) {
    const int r = r0 + (tid >> 4);
    const uint32_t m = mB + r;
    const bool live = r < R && m < p.M;            // whole 16-lane groups agree, so the shuffles below are safe
    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (r < R) {
      const f32x4 *src = (const f32x4 *)(C + r * ldc + g * 8);
      f32x4 a0 = src[0], a1 = src[1];
      v[0] = a0.x; v[1] = a0.y; v[2] = a0.z; v[3] = a0.w; v[4] = a1.x; v[5] = a1.y; v[6] = a1.z; v[7] = a1.w;
    }
    if (epi == E_ONORMGATE) {                                                      // gemm.js:227-232
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; j++) ss += v[j] * v[j];
      ss = sum16(ss);
      const float inv = __frsqrt_rn(ss / 128.0f + p.eps);
      const uint32_t col = nB + g * 8;
      if (live && col < p.N) {
        const uint16_t *gt = p.GT + (size_t)m * p.Ltot + p.ny0 + col;
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = v[j] * inv * p.EV[p.evOff + g * 8 + j] * sigmoid(h_val(gt[j]));
        store_f16x8(p.Y, (size_t)m * p.ldy + p.ny0 + col, v, p.N - col);
      }
      continue;
    }
    // f16 / f32 / bias / resadd (gemm.js:194-203, 211-215)
    const uint32_t col = nB + g * 8;
    if (!live || col >= p.N) continue;
    const uint32_t nv = p.N - col;
    const size_t yi = (size_t)m * p.ldy + p.ny0 + col;
    if (epi == E_F16) {
      store_f16x8(p.Y, yi, v, nv);
    } else if (epi == E_F32) {
      float *y = (float *)p.Y + yi;
      if (nv >= 8 && (((uintptr_t)y) & 15u) == 0) {
        ((f32x4 *)y)[0] = (f32x4){v[0], v[1], v[2], v[3]};
        ((f32x4 *)y)[1] = (f32x4){v[4], v[5], v[6], v[7]};
      } else {
        for (uint32_t j = 0; j < 8 && j < nv; j++) y[j] = v[j];
      }
    } else if (epi == E_BIAS) {                                                   // f16(acc + b[n] (+ Y))
      const float *b = p.EV + p.evOff + col;
      const uint16_t *yh = (const uint16_t *)p.Y + yi;
      const bool res = p.flags & F_RES;
      if (nv >= 8 && (((uintptr_t)yh) & 15u) == 0) {                 // whole 16-byte groups: one residual load
        const u32x4 r = res ? *(const u32x4 *)yh : (u32x4){0u, 0u, 0u, 0u};
        const uint32_t rw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int j = 0; j < 8; j++) {
          float t = v[j] + b[j];
          if (res) t += h_val((uint16_t)(rw[j >> 1] >> (16 * (j & 1))));
          v[j] = t;
        }
      } else {
        for (uint32_t j = 0; j < 8 && j < nv; j++) {
          float t = v[j] + b[j];
          if (res) t += h_val(yh[j]);
          v[j] = t;
        }
      }
      store_f16x8(p.Y, yi, v, nv);
    } else {                                                                       // R += gate[n] * (acc + bias[n])
      float *y = (float *)p.Y + yi;
      const bool gate = p.flags & F_GATE, bias = p.flags & F_BIAS, st = p.flags & F_STORE;
      float gv[8], bv[8];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        gv[j] = (gate && (uint32_t)j < nv) ? p.EV[p.evOff + col + j] : 1.0f;
        bv[j] = (bias && (uint32_t)j < nv) ? p.BV[p.bvOff + col + j] : 0.0f;
      }
      if (nv >= 8 && (((uintptr_t)y) & 15u) == 0) {
        f32x4 p0 = st ? (f32x4){0, 0, 0, 0} : ((const f32x4 *)y)[0], p1 = st ? (f32x4){0, 0, 0, 0} : ((const f32x4 *)y)[1];
        ((f32x4 *)y)[0] = (f32x4){p0.x + gv[0] * (v[0] + bv[0]), p0.y + gv[1] * (v[1] + bv[1]), p0.z + gv[2] * (v[2] + bv[2]),
                                  p0.w + gv[3] * (v[3] + bv[3])};
        ((f32x4 *)y)[1] = (f32x4){p1.x + gv[4] * (v[4] + bv[4]), p1.y + gv[5] * (v[5] + bv[5]), p1.z + gv[6] * (v[6] + bv[6]),
                                  p1.w + gv[7] * (v[7] + bv[7])};
      } else {
        for (uint32_t j = 0; j < 8 && j < nv; j++) y[j] = (st ? 0.0f : y[j]) + gv[j] * (v[j] + bv[j]);
      }
    }
  }
}

}  // namespace p0k
