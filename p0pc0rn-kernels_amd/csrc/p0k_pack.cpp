// p0k_pack.cpp — the weight encoders of docs/FORMAT.md on the host CPU (src/convert/encode.js:56-95): fp32 rows ->
// q4g32a.t64 / q8g64s.t64 records or fp16. These are what a converter or a test bench uses to produce the bytes the
// kernels read; the quantisers follow FORMAT.md exactly: fp32 arithmetic with one rounding per operation, scale and
// minimum rounded to fp16, codes rounded half to even. Rows of 64 are independent, so they encode on several threads.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/p0k.h"

#pragma clang fp contract(off)

namespace {

uint16_t to_half(float v) {   // IEEE binary16, round to nearest even (src/core/gpu.js:276-291)
  uint32_t x;
  std::memcpy(&x, &v, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, ex = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (ex == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
  const int e = (int)ex - 112;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000u;
    const uint32_t sh = (uint32_t)(14 - e), keep = man >> sh, rem = man & ((1u << sh) - 1u), half = 1u << (sh - 1u);
    return (uint16_t)(sign | (keep + ((rem > half || (rem == half && (keep & 1u))) ? 1u : 0u)));
  }
  const uint32_t base = sign | ((uint32_t)e << 10) | (man >> 13), rem = man & 0x1fffu;
  return (uint16_t)(base + ((rem > 0x1000u || (rem == 0x1000u && (base & 1u))) ? 1u : 0u));
}

float from_half(uint16_t h) {
  const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) { bits = s; } else {          // subnormal: m * 2^-24 is exact in fp32
      float f = (float)m * 5.9604644775390625e-8f;
      std::memcpy(&bits, &f, 4);
      bits |= s;
    }
  } else if (e == 31) {
    bits = s | 0x7f800000u | (m << 13);
  } else {
    bits = s | ((e + 112) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

inline float round_half(float v) { return from_half(to_half(v)); }
inline float rne(float v) { return std::nearbyint(v); }   // the default rounding mode: half to even

template <class F>
void parallel_tiles(uint32_t tiles, F fn) {
  unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  nt = std::min<unsigned>(nt, tiles);
  if (nt <= 1) { for (uint32_t t = 0; t < tiles; t++) fn(t); return; }
  std::vector<std::thread> th;
  for (unsigned i = 0; i < nt; i++)
    th.emplace_back([&, i] { for (uint32_t t = i; t < tiles; t += nt) fn(t); });
  for (auto &x : th) x.join();
}

}  // namespace

extern "C" {

uint64_t p0k_tensor_bytes(int enc, uint32_t rows, uint32_t cols) {
  if (enc == P0K_ENC_Q4G32A_T64) return (uint64_t)(rows / 64) * (cols / 32) * 1280u;
  if (enc == P0K_ENC_Q8G64S_T64) return (uint64_t)(rows / 64) * (cols / 64) * 4224u;
  if (enc == P0K_ENC_F16) return (uint64_t)rows * cols * 2u;
  return 0;
}

int p0k_pack_q4(const float *W, uint32_t rows, uint32_t K, uint8_t *out, float *deq) {
  if (!W || !out || rows % 64 || K % 32) return P0K_E_ARG;
  const uint32_t G = K / 32;
  parallel_tiles(rows / 64, [&](uint32_t t) {
    for (uint32_t g = 0; g < G; g++) {
      uint8_t *rec = out + ((uint64_t)t * G + g) * 1280u;
      for (uint32_t r = 0; r < 64; r++) {
        const float *v = W + (uint64_t)(t * 64 + r) * K + (uint64_t)g * 32;
        float lo = INFINITY, hi = -INFINITY;
        for (int i = 0; i < 32; i++) { lo = v[i] < lo ? v[i] : lo; hi = v[i] > hi ? v[i] : hi; }
        const float mn = round_half(lo);
        float s = round_half((hi - mn) / 15.0f);
        if (s == 0.0f) s = 1.0f;
        uint8_t q[32];
        for (int i = 0; i < 32; i++) {
          float c = rne((v[i] - mn) / s);
          q[i] = (uint8_t)(c < 0.0f ? 0 : c > 15.0f ? 15 : (int)c);
          if (deq) deq[(uint64_t)(t * 64 + r) * K + g * 32 + i] = (float)((double)q[i] * s + mn);
        }
        for (int j = 0; j < 16; j++) rec[r * 16 + j] = (uint8_t)(q[2 * j] | (q[2 * j + 1] << 4));
        const uint32_t word = (uint32_t)to_half(s) | ((uint32_t)to_half(mn) << 16);
        std::memcpy(rec + 1024 + r * 4, &word, 4);   // little-endian host
      }
    }
  });
  return P0K_OK;
}

int p0k_pack_q8(const float *W, uint32_t rows, uint32_t K, uint8_t *out, float *deq) {
  if (!W || !out || rows % 64 || K % 64) return P0K_E_ARG;
  const uint32_t G = K / 64;
  parallel_tiles(rows / 64, [&](uint32_t t) {
    for (uint32_t g = 0; g < G; g++) {
      uint8_t *rec = out + ((uint64_t)t * G + g) * 4224u;
      for (uint32_t r = 0; r < 64; r++) {
        const float *v = W + (uint64_t)(t * 64 + r) * K + (uint64_t)g * 64;
        float am = 0.0f;
        for (int i = 0; i < 64; i++) am = std::fabs(v[i]) > am ? std::fabs(v[i]) : am;
        float s = round_half(am / 127.0f);
        if (s == 0.0f) s = 1.0f;
        for (int i = 0; i < 64; i++) {
          float c = rne(v[i] / s);
          int q = c < -128.0f ? -128 : c > 127.0f ? 127 : (int)c;
          rec[r * 64 + i] = (uint8_t)(q & 255);
          if (deq) deq[(uint64_t)(t * 64 + r) * K + g * 64 + i] = (float)((double)q * s);
        }
        const uint16_t sh = to_half(s);
        std::memcpy(rec + 4096 + r * 2, &sh, 2);
      }
    }
  });
  return P0K_OK;
}

int p0k_pack_f16(const float *W, uint64_t n, uint16_t *out) {
  if ((!W || !out) && n) return P0K_E_ARG;
  for (uint64_t i = 0; i < n; i++) out[i] = to_half(W[i]);
  return P0K_OK;
}

}  // extern "C"
