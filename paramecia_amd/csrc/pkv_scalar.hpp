// Scalar helpers shared by host and device code of libpkv.
//
// The Q4K/Q8_0 quantizers must reproduce the bytes of candle's CPU codecs
// (BlockQ4K::from_float / BlockQ8_0::from_float, called from
// paramecia-model/src/qwen3_next.rs:486-487), so the arithmetic here follows Rust
// semantics exactly: f32::round (half away from zero), saturating `as` casts,
// maxNum that drops NaN, and the `half` crate's round-to-nearest-even f16.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/pkv.h"

#define PKV_HD __host__ __device__ __forceinline__

namespace pkv {

PKV_HD uint32_t f2u(float x) { return __builtin_bit_cast(uint32_t, x); }
PKV_HD float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// `v as i32` for an already-rounded v: saturating, NaN -> 0. Written as selects (no
// branches) so that GPU code stays straight-line.
PKV_HD int32_t rs_as_i32(float v) {
  const float c = v > -2147483648.0f ? (v < 2147483520.0f ? v : 2147483520.0f) : -2147483648.0f;
  int32_t r = (int32_t)c;  // c is NaN-free only if v is; the selects below fix the rest
  r = v >= 2147483648.0f ? INT32_MAX : r;
  r = v != v ? 0 : r;
  return r;
}
PKV_HD int32_t rs_as_i8(float v) {
  const float c = v > -128.0f ? (v < 127.0f ? v : 127.0f) : -128.0f;
  return v != v ? 0 : (int32_t)c;
}
// candle's nearest_int: v.round() as i32.
PKV_HD int32_t nearest_int(float v) { return rs_as_i32(__builtin_roundf(v)); }

// f32::total_cmp ordering key.
PKV_HD int32_t total_key(float x) {
  int32_t k = (int32_t)f2u(x);
  k ^= (int32_t)(((uint32_t)(k >> 31)) >> 1);
  return k;
}
// maxNum/minNum: a NaN operand loses; +0 beats -0 for max, -0 beats +0 for min.
// Selects only (no branches).
PKV_HD float fmax_rs(float a, float b) {
  const float gt = a > b ? a : b;                        // a NaN -> b
  const float eq = (f2u(a) & 0x80000000u) ? b : a;       // equal: prefer the non-negative
  const float r = a == b ? eq : gt;
  return a != a ? b : (b != b ? a : r);                   // a NaN -> b, else b NaN -> a
}
PKV_HD float fmin_rs(float a, float b) {
  const float lt = a < b ? a : b;
  const float eq = (f2u(a) & 0x80000000u) ? a : b;       // equal: prefer the negative
  const float r = a == b ? eq : lt;
  return a != a ? b : (b != b ? a : r);
}

// half::f16::from_f32 (round to nearest even, overflow -> inf, quiet NaN), computed
// as selects over the normal, subnormal and special cases (no branches).
PKV_HD uint16_t f32_to_f16(float value) {
  const uint32_t x = f2u(value);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t exp = (x >> 23) & 0xFFu, man = x & 0x007FFFFFu;
  const int32_t he = (int32_t)exp - 112;  // biased f16 exponent
  // normal: truncate, then round to nearest even on the 13 dropped bits (a carry may
  // ripple into the exponent, up to infinity)
  const uint32_t nrm = (((uint32_t)(he & 0x1F) << 10) | (man >> 13)) +
                       (((x & 0x1000u) != 0u && (x & 0x2FFFu) != 0u) ? 1u : 0u);
  // subnormal (he <= 0): shift the implicit-1 mantissa right by 14 - he, same rounding
  const int32_t sh_i = 14 - he;
  const uint32_t sh = (uint32_t)(sh_i < 1 ? 1 : (sh_i > 31 ? 31 : sh_i));
  const uint32_t m = man | 0x00800000u;
  const uint32_t rb = 1u << (sh - 1u);
  const uint32_t sub = (m >> sh) + (((m & rb) != 0u && (m & (3u * rb - 1u)) != 0u) ? 1u : 0u);
  const uint32_t infnan = 0x7C00u | (man != 0u ? 0x0200u : 0u) | (man >> 13);
  uint32_t out = he <= 0 ? (sh_i > 24 ? 0u : sub) : nrm;
  out = he >= 0x1F ? 0x7C00u : out;
  out = exp == 0xFFu ? infnan : out;
  return (uint16_t)(sign | out);
}
PKV_HD float f16_to_f32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
  const float sub = u2f(sign | f2u((float)man * 5.9604644775390625e-08f));  // exact: man * 2^-24
  const float spec = u2f(sign | 0x7F800000u | (man << 13));
  const float nrm = u2f(sign | ((exp + 112u) << 23) | (man << 13));
  return exp == 0u ? sub : (exp == 0x1Fu ? spec : nrm);
}
// half::bf16::from_f32 (round to nearest even, NaN keeps a quiet bit).
PKV_HD uint16_t f32_to_bf16(float value) {
  uint32_t x = f2u(value);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x0040u);
  if ((x & 0x00008000u) != 0 && (x & 0x00017FFFu) != 0) return (uint16_t)((x >> 16) + 1u);
  return (uint16_t)(x >> 16);
}
PKV_HD float bf16_to_f32(uint16_t h) { return u2f(((uint32_t)h) << 16); }

// Philox4x32-10 (Salmon et al., SC'11).
PKV_HD void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
    uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
    uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
    uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
    c[1] = (uint32_t)p1;
    c[3] = (uint32_t)p0;
    c[0] = n0;
    c[2] = n2;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}
// Approximately standard normal: centred sum of eight 22-bit uniforms, scaled by
// sqrt(6)*2^-23 (unit variance). Integer work plus one correctly rounded multiply,
// hence identical on CPU and GPU.
PKV_HD float seeded_normal(uint64_t seed, uint64_t stream, uint64_t index) {
  uint64_t c = 2 * index;
  uint32_t a[4] = {(uint32_t)c, (uint32_t)(c >> 32), (uint32_t)stream, (uint32_t)(stream >> 32)};
  uint32_t b[4] = {(uint32_t)(c + 1), (uint32_t)((c + 1) >> 32), (uint32_t)stream,
                   (uint32_t)(stream >> 32)};
  philox4x32_10(a, (uint32_t)seed, (uint32_t)(seed >> 32));
  philox4x32_10(b, (uint32_t)seed, (uint32_t)(seed >> 32));
  uint32_t s = (a[0] >> 10) + (a[1] >> 10) + (a[2] >> 10) + (a[3] >> 10) + (b[0] >> 10) +
               (b[1] >> 10) + (b[2] >> 10) + (b[3] >> 10);
  return (float)((int32_t)s - (1 << 24)) * 0x1.3988e2p-22f;
}

// Element e of a packed row (candle BlockQ4K/BlockQ8_0::to_float, f16/bf16 widening).
// Callers that need the reference's exact f32 bytes compile with contraction off.
PKV_HD float decode_elem(int quant, const uint8_t *row, int e) {
  switch (quant) {
    case PKV_QUANT_Q4K: {
      const uint8_t *blk = row + (e >> 8) * 144;
      const int w = e & 255, c = w >> 6, l = w & 31, hi = (w >> 5) & 1;
      const int is = 2 * c + hi;
      const uint8_t *s = blk + 4;
      uint32_t sc, m;
      if (is < 4) {
        sc = s[is] & 63;
        m = s[is + 4] & 63;
      } else {
        sc = (s[is + 4] & 0xF) | ((s[is - 4] >> 6) << 4);
        m = (s[is + 4] >> 4) | ((s[is] >> 6) << 4);
      }
      const float d = f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
      const float dmin = f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
      const uint8_t qb = blk[16 + 32 * c + l];
      const uint32_t q = hi ? (qb >> 4) : (qb & 0xF);
      const float d1 = d * (float)sc, m1 = dmin * (float)m;
      return d1 * (float)q - m1;
    }
    case PKV_QUANT_Q8_0: {
      const uint8_t *blk = row + (e >> 5) * 34;
      const float d = f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
      return (float)(int8_t)blk[2 + (e & 31)] * d;
    }
    case PKV_QUANT_BF16:
      return bf16_to_f32(reinterpret_cast<const uint16_t *>(row)[e]);
    default:
      return f16_to_f32(reinterpret_cast<const uint16_t *>(row)[e]);
  }
}

}  // namespace pkv
