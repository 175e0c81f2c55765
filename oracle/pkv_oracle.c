/*
 * pkv_oracle.c — CPU restatement of paramecia-model's quantized KV-cache path.
 * TEST INFRASTRUCTURE ONLY (the checker, never the product). Parity notes per
 * function are in pkv_oracle.h. Built with -ffp-contract=off so that every
 * a*b+c rounds twice, as Rust code does.
 */
#include "pkv_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* Rust scalar semantics                                                */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* `f as i32`: saturating, NaN -> 0. */
static int32_t rust_f32_as_i32(float v) {
  if (v != v) return 0;
  if (v >= 2147483648.0f) return INT32_MAX;
  if (v <= -2147483648.0f) return INT32_MIN;
  return (int32_t)v;
}
/* `f as i8`: saturating, NaN -> 0. */
static int8_t rust_f32_as_i8(float v) {
  if (v != v) return 0;
  if (v >= 127.0f) return 127;
  if (v <= -128.0f) return -128;
  return (int8_t)v;
}
/* candle's nearest_int(v) = v.round() as i32 (round half away from zero). */
static int32_t nearest_int(float v) { return rust_f32_as_i32(roundf(v)); }

/* f32::total_cmp ordering key. */
static int32_t total_key(float x) {
  int32_t k = (int32_t)f2u(x);
  k ^= (int32_t)(((uint32_t)(k >> 31)) >> 1);
  return k;
}

/* IEEE maxNum / minNum (NaN loses). Between +0 and -0 the result is taken as +0 for
 * max and -0 for min; Rust leaves that choice unspecified (see pkv_oracle.h). */
static float fmax_rs(float a, float b) {
  if (a != a) return b;
  if (b != b) return a;
  if (a > b) return a;
  if (b > a) return b;
  return (f2u(a) & 0x80000000u) ? b : a; /* equal: prefer +0 over -0 */
}
static float fmin_rs(float a, float b) {
  if (a != a) return b;
  if (b != b) return a;
  if (a < b) return a;
  if (b < a) return b;
  return (f2u(a) & 0x80000000u) ? a : b; /* equal: prefer -0 over +0 */
}

/* ------------------------------------------------------------------ */
/* half crate conversions                                               */
/* ------------------------------------------------------------------ */

uint16_t orc_f32_to_f16(float value) {
  uint32_t x = f2u(value);
  uint32_t sign = x & 0x80000000u;
  uint32_t exp = x & 0x7F800000u;
  uint32_t man = x & 0x007FFFFFu;
  if (exp == 0x7F800000u) { /* inf / NaN (NaN keeps a quiet payload bit) */
    uint32_t nan_bit = (man == 0) ? 0 : 0x0200u;
    return (uint16_t)((sign >> 16) | 0x7C00u | nan_bit | (man >> 13));
  }
  uint32_t half_sign = sign >> 16;
  int32_t unbiased = ((int32_t)(exp >> 23)) - 127;
  int32_t half_exp = unbiased + 15;
  if (half_exp >= 0x1F) return (uint16_t)(half_sign | 0x7C00u); /* overflow -> inf */
  if (half_exp <= 0) {                                            /* subnormal / zero */
    if (14 - half_exp > 24) return (uint16_t)half_sign;
    uint32_t m = man | 0x00800000u;
    uint32_t shift = (uint32_t)(14 - half_exp);
    uint32_t half_man = m >> shift;
    uint32_t round_bit = 1u << (shift - 1);
    if ((m & round_bit) != 0 && (m & (3u * round_bit - 1u)) != 0) half_man++;
    return (uint16_t)(half_sign | half_man);
  }
  uint32_t half_e = ((uint32_t)half_exp) << 10;
  uint32_t half_man = man >> 13;
  uint32_t round_bit = 0x00001000u;
  if ((x & round_bit) != 0 && (x & (3u * round_bit - 1u)) != 0)
    return (uint16_t)((half_sign | half_e | half_man) + 1u); /* carry may reach inf */
  return (uint16_t)(half_sign | half_e | half_man);
}

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  if (exp == 0) {
    if (man == 0) return u2f(sign);
    /* subnormal: value = man * 2^-24, exact in f32 */
    float v = (float)man * 5.9604644775390625e-08f;
    return (sign ? -v : v);
  }
  if (exp == 0x1F) return u2f(sign | 0x7F800000u | (man << 13));
  return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t orc_f32_to_bf16(float value) {
  uint32_t x = f2u(value);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x0040u);
  uint32_t round_bit = 0x00008000u;
  if ((x & round_bit) != 0 && (x & (3u * round_bit - 1u)) != 0)
    return (uint16_t)((x >> 16) + 1u);
  return (uint16_t)(x >> 16);
}

float orc_bf16_to_f32(uint16_t h) { return u2f(((uint32_t)h) << 16); }

void orc_f32_to_f16_n(const float *x, uint16_t *out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16(x[i]);
}
void orc_f32_to_bf16_n(const float *x, uint16_t *out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(x[i]);
}
void orc_f16_to_f32_n(const uint16_t *h, float *out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32(h[i]);
}

/* ------------------------------------------------------------------ */
/* Q8_0: { f16 d; i8 qs[32]; } = 34 bytes                              */
/* ------------------------------------------------------------------ */

void orc_q8_0_quantize(const float *x, uint8_t *out, size_t n) {
  for (size_t b = 0; b < n / 32; ++b) {
    const float *xs = x + 32 * b;
    uint8_t *blk = out + 34 * b;
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = fmax_rs(amax, fabsf(xs[i]));
    float d = amax / 127.0f;
    float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    uint16_t dh = orc_f32_to_f16(d);
    blk[0] = (uint8_t)(dh & 0xFF);
    blk[1] = (uint8_t)(dh >> 8);
    for (int i = 0; i < 32; ++i) blk[2 + i] = (uint8_t)rust_f32_as_i8(roundf(xs[i] * id));
  }
}

void orc_q8_0_dequantize(const uint8_t *in, float *y, size_t n) {
  for (size_t b = 0; b < n / 32; ++b) {
    const uint8_t *blk = in + 34 * b;
    float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    for (int i = 0; i < 32; ++i) y[32 * b + i] = (float)(int8_t)blk[2 + i] * d;
  }
}

/* ------------------------------------------------------------------ */
/* Q4K: { f16 d; f16 dmin; u8 scales[12]; u8 qs[128]; } = 144 bytes    */
/* ------------------------------------------------------------------ */

/* ORC_MUTANT plants one mistake in make_qkx1_quants, for tests/test_oracle_mutants.py
 * only (the normal build leaves it 0): 1 one pass fewer, 2 one pass more, 3 no early
 * exit, 4 ties rounded to even, 5 pairwise (tree) sums instead of sequential ones,
 * 6 GGML's make_qkx2_quants in its place, 7 no `min > 0 -> 0` clamp inside the loop. */
#ifndef ORC_MUTANT
#define ORC_MUTANT 0
#endif
#if ORC_MUTANT == 5
static float tree_sum(float *t, int n) {
  for (int w = 1; w < n; w *= 2)
    for (int i = 0; i + w < n; i += 2 * w) t[i] = t[i] + t[i + w];
  return n > 0 ? t[0] : 0.0f;
}
#endif
#if ORC_MUTANT == 6
/* GGML make_qkx2_quants as quantize_row_q4_K_ref calls it: weights av_x + |x|,
 * rmin -1, rdelta 0.1, nstep 20, squared error. */
static void qkx2_mutant(const float *x, int n, int nmax, float *scale_out, float *neg_min_out) {
  float w[256], sum_x2 = 0.0f;
  for (int i = 0; i < n; ++i) sum_x2 += x[i] * x[i];
  const float av_x = sqrtf(sum_x2 / n);
  for (int i = 0; i < n; ++i) w[i] = av_x + fabsf(x[i]);
  float mn = x[0], mx = x[0], sum_w = w[0], sum_x = w[0] * x[0];
  for (int i = 1; i < n; ++i) {
    if (x[i] < mn) mn = x[i];
    if (x[i] > mx) mx = x[i];
    sum_w += w[i];
    sum_x += w[i] * x[i];
  }
  if (mn > 0) mn = 0;
  if (mx == mn) {
    *scale_out = 0.0f;
    *neg_min_out = -mn;
    return;
  }
  float iscale = nmax / (mx - mn), scale = 1.0f / iscale, best = 0.0f;
  for (int i = 0; i < n; ++i) {
    int l = nearest_int(iscale * (x[i] - mn));
    l = l < 0 ? 0 : (l > nmax ? nmax : l);
    const float d = scale * l + mn - x[i];
    best += w[i] * d * d;
  }
  for (int is = 0; is <= 20; ++is) {
    iscale = (-1.0f + 0.1f * is + nmax) / (mx - mn);
    float sl = 0, sl2 = 0, sxl = 0;
    uint8_t La[256];
    for (int i = 0; i < n; ++i) {
      int l = nearest_int(iscale * (x[i] - mn));
      l = l < 0 ? 0 : (l > nmax ? nmax : l);
      La[i] = (uint8_t)l;
      sl += w[i] * l;
      sl2 += w[i] * l * l;
      sxl += w[i] * l * x[i];
    }
    const float D = sum_w * sl2 - sl * sl;
    if (D > 0) {
      float ts = (sum_w * sxl - sum_x * sl) / D, tm = (sl2 * sum_x - sl * sxl) / D;
      if (tm > 0) {
        tm = 0;
        ts = sxl / sl2;
      }
      float mad = 0;
      for (int i = 0; i < n; ++i) {
        const float d = ts * La[i] + tm - x[i];
        mad += w[i] * d * d;
      }
      if (mad < best) {
        best = mad;
        scale = ts;
        mn = tm;
      }
    }
  }
  *scale_out = scale;
  *neg_min_out = -mn;
}
#endif

void orc_make_qkx1_quants(const float *x, int n, int nmax, int ntry, float *scale_out,
                          float *neg_min_out) {
#if ORC_MUTANT == 6
  qkx2_mutant(x, n, nmax, scale_out, neg_min_out);
  return;
#endif
#if ORC_MUTANT == 1
  ntry -= 1;
#elif ORC_MUTANT == 2
  ntry += 1;
#endif
  uint8_t L[256];
  memset(L, 0, sizeof(L));
  float mn = x[0], mx = x[0];
  for (int i = 1; i < n; ++i) {
    if (total_key(x[i]) < total_key(mn)) mn = x[i];
    if (total_key(x[i]) >= total_key(mx)) mx = x[i];
  }
  if (mx == mn) {
    *scale_out = 0.0f;
    *neg_min_out = 0.0f;
    return;
  }
  float min = fmin_rs(mn, 0.0f);
  float iscale = (float)nmax / (mx - min);
  float scale = 1.0f / iscale;
  for (int t = 0; t < ntry; ++t) {
    float sumlx = 0.0f;
    int32_t suml2 = 0;
    int did_change = 0;
#if ORC_MUTANT == 5
    float terms[256];
#endif
    for (int i = 0; i < n; ++i) {
#if ORC_MUTANT == 4
      int32_t li = rust_f32_as_i32(rintf(iscale * (x[i] - min)));
#else
      int32_t li = nearest_int(iscale * (x[i] - min));
#endif
      if (li < 0) li = 0;
      if (li > nmax) li = nmax;
      if ((uint8_t)li != L[i]) {
        L[i] = (uint8_t)li;
        did_change = 1;
      }
#if ORC_MUTANT == 5
      terms[i] = (x[i] - min) * (float)li;
#else
      sumlx += (x[i] - min) * (float)li;
#endif
      suml2 += li * li;
    }
#if ORC_MUTANT == 5
    sumlx = tree_sum(terms, n);
#endif
    scale = sumlx / (float)suml2;
    float sum = -0.0f;
#if ORC_MUTANT == 5
    for (int i = 0; i < n; ++i) terms[i] = x[i] - scale * (float)L[i];
    sum = tree_sum(terms, n);
#else
    for (int i = 0; i < n; ++i) sum += x[i] - scale * (float)L[i];
#endif
    min = sum / (float)n;
#if ORC_MUTANT != 7
    if (min > 0.0f) min = 0.0f;
#endif
    iscale = 1.0f / scale;
#if ORC_MUTANT != 3
    if (!did_change) break;
#endif
  }
  *scale_out = scale;
  *neg_min_out = -min;
}

void orc_get_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

static void q4k_quantize_block(const float *x, uint8_t *blk) {
  float mins[8], scales[8];
  uint8_t *sc = blk + 4, *qs = blk + 16;
  memset(blk, 0, 144);
  for (int j = 0; j < 8; ++j) orc_make_qkx1_quants(x + 32 * j, 32, 15, 5, &scales[j], &mins[j]);
  float max_scale = 0.0f, max_min = 0.0f;
  for (int j = 0; j < 8; ++j) {
    max_scale = fmax_rs(scales[j], max_scale);
    max_min = fmax_rs(mins[j], max_min);
  }
  float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
  float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
  for (int j = 0; j < 8; ++j) {
    int32_t ls32 = nearest_int(inv_scale * scales[j]);
    int32_t lm32 = nearest_int(inv_min * mins[j]);
    uint8_t ls = (uint8_t)(ls32 < 63 ? ls32 : 63);
    uint8_t lm = (uint8_t)(lm32 < 63 ? lm32 : 63);
    if (j < 4) {
      sc[j] = ls;
      sc[j + 4] = lm;
    } else {
      sc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
      sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
      sc[j] |= (uint8_t)((lm >> 4) << 6);
    }
  }
  uint16_t dh = orc_f32_to_f16(max_scale / 63.0f);
  uint16_t mh = orc_f32_to_f16(max_min / 63.0f);
  blk[0] = (uint8_t)(dh & 0xFF);
  blk[1] = (uint8_t)(dh >> 8);
  blk[2] = (uint8_t)(mh & 0xFF);
  blk[3] = (uint8_t)(mh >> 8);
  float d_all = orc_f16_to_f32(dh), m_all = orc_f16_to_f32(mh);
  uint8_t L[256];
  memset(L, 0, sizeof(L));
  for (int j = 0; j < 8; ++j) {
    uint8_t s, m;
    orc_get_scale_min_k4(j, sc, &s, &m);
    float d = d_all * (float)s;
    if (d != 0.0f) {
      float dm = m_all * (float)m;
      for (int ii = 0; ii < 32; ++ii) {
        int32_t l = nearest_int((x[32 * j + ii] + dm) / d);
        if (l < 0) l = 0;
        if (l > 15) l = 15;
        L[32 * j + ii] = (uint8_t)l;
      }
    }
  }
  for (int j = 0; j < 256; j += 64)
    for (int l = 0; l < 32; ++l) qs[(j / 64) * 32 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
}

void orc_q4k_quantize(const float *x, uint8_t *out, size_t n) {
  for (size_t b = 0; b < n / 256; ++b) q4k_quantize_block(x + 256 * b, out + 144 * b);
}

void orc_q4k_dequantize(const uint8_t *in, float *y, size_t n) {
  for (size_t b = 0; b < n / 256; ++b) {
    const uint8_t *blk = in + 144 * b;
    float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    float min = orc_f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
    const uint8_t *sc = blk + 4, *qs = blk + 16;
    float *yb = y + 256 * b;
    int is = 0, yi = 0;
    for (int j = 0; j < 256; j += 64) {
      const uint8_t *q = qs + j / 2;
      uint8_t s, m;
      orc_get_scale_min_k4(is, sc, &s, &m);
      float d1 = d * (float)s, m1 = min * (float)m;
      orc_get_scale_min_k4(is + 1, sc, &s, &m);
      float d2 = d * (float)s, m2 = min * (float)m;
      for (int l = 0; l < 32; ++l) yb[yi++] = d1 * (float)(q[l] & 0xF) - m1;
      for (int l = 0; l < 32; ++l) yb[yi++] = d2 * (float)(q[l] >> 4) - m2;
      is += 2;
    }
  }
}

/* GGUF Q5_K: 176-byte superblocks {f16 d, f16 dmin, 12 B 6-bit scale/min codes (the Q4K
 * packing), 32 B high bits qh, 128 B low nibbles qs}. Element 64 c + l (c = 0..3, l < 32)
 * takes the low nibble of qs[32 c + l] plus 16 if bit 2 c of qh[l] is set, scaled by
 * sub-block 2 c; element 64 c + 32 + l takes the high nibble plus bit 2 c + 1, scaled by
 * sub-block 2 c + 1. y = (d * sc) * code - dmin * m in f32 (upstream candle k_quants.rs
 * BlockQ5K::to_float; ggml dequantize_row_q5_K). */
void orc_q5k_dequantize(const uint8_t *in, float *y, size_t n) {
  for (size_t b = 0; b < n / 256; ++b) {
    const uint8_t *blk = in + 176 * b;
    const float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    const float min = orc_f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
    const uint8_t *sc = blk + 4, *qh = blk + 16, *qs = blk + 48;
    float *yb = y + 256 * b;
    for (int c = 0; c < 4; ++c) {
      uint8_t s, m;
      orc_get_scale_min_k4(2 * c, sc, &s, &m);
      const float d1 = d * (float)s, m1 = min * (float)m;
      orc_get_scale_min_k4(2 * c + 1, sc, &s, &m);
      const float d2 = d * (float)s, m2 = min * (float)m;
      const uint8_t u1 = (uint8_t)(1u << (2 * c)), u2 = (uint8_t)(2u << (2 * c));
      for (int l = 0; l < 32; ++l) {
        const float add = (qh[l] & u1) ? 16.0f : 0.0f;
        yb[64 * c + l] = d1 * ((float)(qs[32 * c + l] & 0xF) + add) - m1;
      }
      for (int l = 0; l < 32; ++l) {
        const float add = (qh[l] & u2) ? 16.0f : 0.0f;
        yb[64 * c + 32 + l] = d2 * ((float)(qs[32 * c + l] >> 4) + add) - m2;
      }
    }
  }
}

/* GGUF Q6_K: 210-byte superblocks {128 B low nibbles ql, 64 B high bit pairs qh, 16 int8
 * scales, f16 d (last)}. In half h (elements 128 h ..) with l < 32: groups g = 0..3 hold
 * elements 128 h + 32 g + l; the low 4 bits come from ql[64 h + l + 32 (g & 1)] (low
 * nibble for g < 2, high for g >= 2), bits 4-5 from bits 2 g, 2 g + 1 of qh[32 h + l];
 * the signed code is that minus 32, scaled by scales[8 h + 2 g + l / 16], which is
 * scales[e / 16] for element e. y = (d * sc) * q in f32 (upstream candle k_quants.rs
 * BlockQ6K::to_float; ggml dequantize_row_q6_K). */
void orc_q6k_dequantize(const uint8_t *in, float *y, size_t n) {
  for (size_t b = 0; b < n / 256; ++b) {
    const uint8_t *blk = in + 210 * b;
    const float d = orc_f16_to_f32((uint16_t)(blk[208] | (blk[209] << 8)));
    float *yb = y + 256 * b;
    for (int h = 0; h < 2; ++h) {
      const uint8_t *ql = blk + 64 * h, *qh = blk + 128 + 32 * h;
      const int8_t *sc = (const int8_t *)(blk + 192 + 8 * h);
      for (int l = 0; l < 32; ++l) {
        const int is = l / 16;
        const int q1 = (int)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
        const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
        const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
        const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
        yb[128 * h + l] = d * (float)sc[is] * (float)q1;
        yb[128 * h + l + 32] = d * (float)sc[is + 2] * (float)q2;
        yb[128 * h + l + 64] = d * (float)sc[is + 4] * (float)q3;
        yb[128 * h + l + 96] = d * (float)sc[is + 6] * (float)q4;
      }
    }
  }
}

/* ------------------------------------------------------------------ */
/* Seeded synthetic data: Philox4x32-10 + Irwin-Hall(8) normal          */
/* ------------------------------------------------------------------ */

void orc_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
  uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
  uint32_t k0 = key_in[0], k1 = key_in[1];
  for (int r = 0; r < 10; ++r) {
    uint64_t p0 = (uint64_t)0xD2511F53u * c0;
    uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
    uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
    uint32_t n1 = (uint32_t)p1;
    uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
    uint32_t n3 = (uint32_t)p0;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* Sum of eight 22-bit uniforms, centred and scaled to unit variance. Every step is an
 * integer operation or one correctly rounded f32 multiply, so the GPU generator
 * (paramecia_amd/csrc) reproduces it bit for bit. */
float orc_normal(uint64_t seed, uint64_t stream, uint64_t index) {
  uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  uint32_t r[8];
  uint64_t c = 2 * index;
  uint32_t ctr[4] = {(uint32_t)c, (uint32_t)(c >> 32), (uint32_t)stream,
                     (uint32_t)(stream >> 32)};
  orc_philox4x32_10(ctr, key, r);
  ctr[0] = (uint32_t)(c + 1);
  ctr[1] = (uint32_t)((c + 1) >> 32);
  orc_philox4x32_10(ctr, key, r + 4);
  uint32_t s = 0;
  for (int i = 0; i < 8; ++i) s += r[i] >> 10;
  return (float)((int32_t)s - (1 << 24)) * 0x1.3988e2p-22f;
}

void orc_fill_normal(float *out, size_t n, uint64_t seed, uint64_t stream, float scale) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_normal(seed, stream, i) * scale;
}

/* ------------------------------------------------------------------ */
/* Preallocated quantized cache (qwen3_next.rs:343-643)                 */
/* ------------------------------------------------------------------ */

static int block_of(int quant) {
  return quant == ORC_Q8_0 ? 32 : quant == ORC_Q4K ? 256 : 1;
}

size_t orc_bytes_per_row(int quant, int head_dim) {
  int bs = block_of(quant);
  int padded = (head_dim + bs - 1) / bs * bs;
  switch (quant) {
    case ORC_Q8_0: return (size_t)(padded / 32) * 34;
    case ORC_Q4K: return (size_t)(padded / 256) * 144;
    case ORC_F16:
    case ORC_BF16: return (size_t)padded * 2;
    default: return 0;
  }
}

int orc_cache_init(orc_cache *c, int quant, int batch, int n_kv_heads, int head_dim,
                   int64_t max_seq_len) {
  memset(c, 0, sizeof(*c));
  if (quant < ORC_F16 || quant > ORC_Q4K || batch <= 0 || n_kv_heads <= 0 || head_dim <= 0 ||
      max_seq_len < 0)
    return ORC_ERR_ARG;
  c->quant = quant;
  c->batch = batch;
  c->n_kv_heads = n_kv_heads;
  c->head_dim = head_dim;
  c->block = block_of(quant);
  c->padded_head_dim = (head_dim + c->block - 1) / c->block * c->block;
  c->max_seq_len = max_seq_len;
  c->bytes_per_row = orc_bytes_per_row(quant, head_dim);
  size_t total = (size_t)batch * n_kv_heads * (size_t)max_seq_len * c->bytes_per_row;
  c->k = (uint8_t *)calloc(total ? total : 1, 1);
  c->v = (uint8_t *)calloc(total ? total : 1, 1);
  return (c->k && c->v) ? ORC_OK : ORC_ERR_ARG;
}

void orc_cache_free(orc_cache *c) {
  free(c->k);
  free(c->v);
  c->k = c->v = NULL;
}

static void encode_row(int quant, const float *x, int padded, uint8_t *dst) {
  switch (quant) {
    case ORC_Q8_0: orc_q8_0_quantize(x, dst, (size_t)padded); break;
    case ORC_Q4K: orc_q4k_quantize(x, dst, (size_t)padded); break;
    case ORC_F16:
      for (int e = 0; e < padded; ++e) {
        uint16_t h = orc_f32_to_f16(x[e]);
        dst[2 * e] = (uint8_t)h;
        dst[2 * e + 1] = (uint8_t)(h >> 8);
      }
      break;
    case ORC_BF16:
      for (int e = 0; e < padded; ++e) {
        uint16_t h = orc_f32_to_bf16(x[e]);
        dst[2 * e] = (uint8_t)h;
        dst[2 * e + 1] = (uint8_t)(h >> 8);
      }
      break;
  }
}

static void decode_row(int quant, const uint8_t *src, int padded, float *y) {
  switch (quant) {
    case ORC_Q8_0: orc_q8_0_dequantize(src, y, (size_t)padded); break;
    case ORC_Q4K: orc_q4k_dequantize(src, y, (size_t)padded); break;
    case ORC_F16:
      for (int e = 0; e < padded; ++e) y[e] = orc_f16_to_f32((uint16_t)(src[2 * e] | (src[2 * e + 1] << 8)));
      break;
    case ORC_BF16:
      for (int e = 0; e < padded; ++e) y[e] = orc_bf16_to_f32((uint16_t)(src[2 * e] | (src[2 * e + 1] << 8)));
      break;
  }
}

int orc_cache_append(orc_cache *c, const float *k, const float *v, int64_t n) {
  if (n < 0) return ORC_ERR_ARG;
  if (c->seq_len + n > c->max_seq_len) return ORC_ERR_OVERFLOW; /* no partial write */
  const int B = c->batch, H = c->n_kv_heads, D = c->head_dim, P = c->padded_head_dim;
  float *row = (float *)calloc((size_t)P, sizeof(float));
  for (int64_t t = 0; t < n; ++t)
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < H; ++h) {
        size_t r = ((size_t)(c->seq_len + t) * B + b) * H + h;
        size_t src = (((size_t)b * H + h) * (size_t)n + (size_t)t) * D;
        for (int p = 0; p < 2; ++p) {
          const float *x = p ? v : k;
          memcpy(row, x + src, (size_t)D * sizeof(float));
          for (int e = D; e < P; ++e) row[e] = 0.0f;
          encode_row(c->quant, row, P, (p ? c->v : c->k) + r * c->bytes_per_row);
        }
      }
  free(row);
  c->seq_len += n;
  return ORC_OK;
}

int orc_cache_append_at(orc_cache *c, const float *k, const float *v, int64_t n,
                        int64_t offset) {
  if (offset != c->seq_len) {
    if (offset <= c->seq_len)
      orc_cache_truncate(c, offset);
    else
      return ORC_ERR_OFFSET;
  }
  return orc_cache_append(c, k, v, n);
}

void orc_cache_truncate(orc_cache *c, int64_t new_len) {
  if (new_len < c->seq_len) c->seq_len = new_len < 0 ? 0 : new_len;
}

void orc_cache_clear(orc_cache *c) { c->seq_len = 0; }

int orc_cache_resize_batch(orc_cache *c, int batch) {
  if (batch <= 0) return ORC_ERR_ARG;
  if (batch != c->batch) {
    int q = c->quant, H = c->n_kv_heads, D = c->head_dim;
    int64_t m = c->max_seq_len;
    orc_cache_free(c);
    return orc_cache_init(c, q, batch, H, D, m);
  }
  return ORC_OK;
}

void orc_cache_get_kv(const orc_cache *c, float *k_out, float *v_out) {
  const int B = c->batch, H = c->n_kv_heads, D = c->head_dim, P = c->padded_head_dim;
  const int64_t S = c->seq_len;
  float *row = (float *)malloc((size_t)P * sizeof(float));
  for (int64_t t = 0; t < S; ++t)
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < H; ++h) {
        size_t r = ((size_t)t * B + b) * H + h;
        size_t dst = (((size_t)b * H + h) * (size_t)S + (size_t)t) * D;
        decode_row(c->quant, c->k + r * c->bytes_per_row, P, row);
        memcpy(k_out + dst, row, (size_t)D * sizeof(float));
        decode_row(c->quant, c->v + r * c->bytes_per_row, P, row);
        memcpy(v_out + dst, row, (size_t)D * sizeof(float));
      }
  free(row);
}

/* ------------------------------------------------------------------ */
/* Attention (qwen3_next.rs:2580-2605)                                  */
/* ------------------------------------------------------------------ */

static int attn_args_ok(const orc_cache *c, int l, int num_heads) {
  return l > 0 && num_heads > 0 && num_heads % c->n_kv_heads == 0;
}

static inline int visible(int64_t j, int i, int64_t q_offset, int masked) {
  return !masked || j <= (int64_t)i + q_offset;
}

int orc_attend_f32(const orc_cache *c, const float *q, int l, int num_heads, float scale,
                   int64_t q_offset, int causal, float *out, int threads) {
  if (!attn_args_ok(c, l, num_heads)) return ORC_ERR_ARG;
  const int B = c->batch, Hkv = c->n_kv_heads, D = c->head_dim, G = num_heads / Hkv;
  const int64_t S = c->seq_len;
  const int masked = causal;
  float *K = (float *)malloc((size_t)B * Hkv * (size_t)S * D * sizeof(float) + 4);
  float *V = (float *)malloc((size_t)B * Hkv * (size_t)S * D * sizeof(float) + 4);
  orc_cache_get_kv(c, K, V);
#ifdef _OPENMP
  int nt = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel for collapse(2) schedule(dynamic) num_threads(nt)
#endif
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < num_heads; ++h) {
      float *s = (float *)malloc((size_t)S * sizeof(float) + 4);
      const float *Kh = K + ((size_t)b * Hkv + h / G) * (size_t)S * D;
      const float *Vh = V + ((size_t)b * Hkv + h / G) * (size_t)S * D;
      for (int i = 0; i < l; ++i) {
        const float *qv = q + (((size_t)b * l + i) * num_heads + h) * D;
        float mx = -INFINITY;
        for (int64_t j = 0; j < S; ++j) {
          float acc = 0.0f;
          for (int e = 0; e < D; ++e) acc += qv[e] * Kh[(size_t)j * D + e];
          acc *= scale;
          if (!visible(j, i, q_offset, masked)) acc = -INFINITY;
          acc = acc < -100.0f ? -100.0f : (acc > 100.0f ? 100.0f : acc);
          s[j] = acc;
          if (acc > mx) mx = acc;
        }
        float sum = 0.0f;
        for (int64_t j = 0; j < S; ++j) {
          s[j] = expf(s[j] - mx);
          sum += s[j];
        }
        float *o = out + (((size_t)b * l + i) * num_heads + h) * D;
        for (int e = 0; e < D; ++e) o[e] = 0.0f;
        for (int64_t j = 0; j < S; ++j) {
          float p = s[j] / sum;
          for (int e = 0; e < D; ++e) o[e] += p * Vh[(size_t)j * D + e];
        }
      }
      free(s);
    }
  free(K);
  free(V);
  (void)threads;
  return ORC_OK;
}

int orc_attend_f64(const orc_cache *c, const float *q, int l, int num_heads, double scale,
                   int64_t q_offset, int causal, double *out) {
  if (!attn_args_ok(c, l, num_heads)) return ORC_ERR_ARG;
  const int B = c->batch, Hkv = c->n_kv_heads, D = c->head_dim, G = num_heads / Hkv;
  const int64_t S = c->seq_len;
  const int masked = causal;
  float *K = (float *)malloc((size_t)B * Hkv * (size_t)S * D * sizeof(float) + 4);
  float *V = (float *)malloc((size_t)B * Hkv * (size_t)S * D * sizeof(float) + 4);
  orc_cache_get_kv(c, K, V);
#ifdef _OPENMP
#pragma omp parallel for collapse(2) schedule(dynamic)
#endif
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < num_heads; ++h) {
      double *s = (double *)malloc((size_t)S * sizeof(double) + 8);
      const float *Kh = K + ((size_t)b * Hkv + h / G) * (size_t)S * D;
      const float *Vh = V + ((size_t)b * Hkv + h / G) * (size_t)S * D;
      for (int i = 0; i < l; ++i) {
        const float *qv = q + (((size_t)b * l + i) * num_heads + h) * D;
        double mx = -INFINITY;
        for (int64_t j = 0; j < S; ++j) {
          double acc = 0.0;
          for (int e = 0; e < D; ++e) acc += (double)qv[e] * (double)Kh[(size_t)j * D + e];
          acc *= scale;
          if (!visible(j, i, q_offset, masked)) acc = -INFINITY;
          acc = acc < -100.0 ? -100.0 : (acc > 100.0 ? 100.0 : acc);
          s[j] = acc;
          if (acc > mx) mx = acc;
        }
        double sum = 0.0;
        for (int64_t j = 0; j < S; ++j) {
          s[j] = exp(s[j] - mx);
          sum += s[j];
        }
        double *o = out + (((size_t)b * l + i) * num_heads + h) * D;
        for (int e = 0; e < D; ++e) o[e] = 0.0;
        for (int64_t j = 0; j < S; ++j) {
          const double p = s[j] / sum;
          for (int e = 0; e < D; ++e) o[e] += p * (double)Vh[(size_t)j * D + e];
        }
      }
      free(s);
    }
  free(K);
  free(V);
  return ORC_OK;
}

int orc_attend_faithful(const orc_cache *c, const float *q, int l, int num_heads,
                        float scale, int64_t q_offset, int causal, float *out, int threads) {
  if (!attn_args_ok(c, l, num_heads)) return ORC_ERR_ARG;
  const int B = c->batch, Hkv = c->n_kv_heads, D = c->head_dim, G = num_heads / Hkv;
  const int64_t S = c->seq_len;
  const int masked = causal;
  const size_t SD = (size_t)S * D;
#ifdef _OPENMP
  int nt = threads > 0 ? threads : omp_get_max_threads();
#else
  int nt = 1;
#endif
  /* get_kv: dequantize the whole valid cache into [S,B,Hkv,P] then permute-copy to
   * [B,Hkv,S,D] (qwen3_next.rs:541-573, .contiguous() at :2471-2472). */
  const int P = c->padded_head_dim;
  float *deq_k = (float *)malloc((size_t)S * B * Hkv * P * sizeof(float) + 4);
  float *deq_v = (float *)malloc((size_t)S * B * Hkv * P * sizeof(float) + 4);
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nt)
#endif
  for (int64_t r = 0; r < S * B * Hkv; ++r) {
    decode_row(c->quant, c->k + (size_t)r * c->bytes_per_row, P, deq_k + (size_t)r * P);
    decode_row(c->quant, c->v + (size_t)r * c->bytes_per_row, P, deq_v + (size_t)r * P);
  }
  float *K = (float *)malloc((size_t)B * Hkv * SD * sizeof(float) + 4);
  float *V = (float *)malloc((size_t)B * Hkv * SD * sizeof(float) + 4);
#ifdef _OPENMP
#pragma omp parallel for collapse(2) schedule(static) num_threads(nt)
#endif
  for (int bh = 0; bh < B * Hkv; ++bh)
    for (int64_t t = 0; t < S; ++t) {
      memcpy(K + (size_t)bh * SD + (size_t)t * D, deq_k + ((size_t)t * B * Hkv + bh) * P, (size_t)D * 4);
      memcpy(V + (size_t)bh * SD + (size_t)t * D, deq_v + ((size_t)t * B * Hkv + bh) * P, (size_t)D * 4);
    }
  free(deq_k);
  free(deq_v);
  /* repeat_kv: materialise [B, H, S, D] for K and V (utils.rs:71-83). */
  float *Kr = (float *)malloc((size_t)B * num_heads * SD * sizeof(float) + 4);
  float *Vr = (float *)malloc((size_t)B * num_heads * SD * sizeof(float) + 4);
#ifdef _OPENMP
#pragma omp parallel for collapse(2) schedule(static) num_threads(nt)
#endif
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < num_heads; ++h) {
      memcpy(Kr + ((size_t)b * num_heads + h) * SD, K + ((size_t)b * Hkv + h / G) * SD, SD * 4);
      memcpy(Vr + ((size_t)b * num_heads + h) * SD, V + ((size_t)b * Hkv + h / G) * SD, SD * 4);
    }
  free(K);
  free(V);
  /* k.transpose(2,3).contiguous(): [B, H, D, S] */
  float *Kt = (float *)malloc((size_t)B * num_heads * SD * sizeof(float) + 4);
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nt)
#endif
  for (int bh = 0; bh < B * num_heads; ++bh)
    for (int64_t t = 0; t < S; ++t)
      for (int e = 0; e < D; ++e)
        Kt[(size_t)bh * SD + (size_t)e * S + t] = Kr[(size_t)bh * SD + (size_t)t * D + e];
  free(Kr);
  /* scores = q.matmul(kT) * scale (+mask), clamp, softmax_last_dim, matmul(v) */
#ifdef _OPENMP
#pragma omp parallel for collapse(2) schedule(dynamic) num_threads(nt)
#endif
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < num_heads; ++h) {
      const size_t bh = (size_t)b * num_heads + h;
      float *sc = (float *)malloc((size_t)l * S * sizeof(float) + 4);
      for (int i = 0; i < l; ++i) {
        const float *qv = q + (((size_t)b * l + i) * num_heads + h) * D;
        float *srow = sc + (size_t)i * S;
        for (int64_t j = 0; j < S; ++j) srow[j] = 0.0f;
        for (int e = 0; e < D; ++e) {
          const float qe = qv[e];
          const float *kt = Kt + bh * SD + (size_t)e * S;
          for (int64_t j = 0; j < S; ++j) srow[j] += qe * kt[j];
        }
        float mx = -INFINITY;
        for (int64_t j = 0; j < S; ++j) {
          float a = srow[j] * scale;
          if (!visible(j, i, q_offset, masked)) a = -INFINITY;
          a = a < -100.0f ? -100.0f : (a > 100.0f ? 100.0f : a);
          srow[j] = a;
          if (a > mx) mx = a;
        }
        float sum = 0.0f;
        for (int64_t j = 0; j < S; ++j) {
          srow[j] = expf(srow[j] - mx);
          sum += srow[j];
        }
        for (int64_t j = 0; j < S; ++j) srow[j] /= sum;
        float *o = out + (((size_t)b * l + i) * num_heads + h) * D;
        for (int e = 0; e < D; ++e) o[e] = 0.0f;
        for (int64_t j = 0; j < S; ++j) {
          const float p = srow[j];
          const float *vr = Vr + bh * SD + (size_t)j * D;
          for (int e = 0; e < D; ++e) o[e] += p * vr[e];
        }
      }
      free(sc);
    }
  free(Kt);
  free(Vr);
  return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* q/k preparation: RMSNorm + partial RoPE (qwen3_next.rs:2369-2399)     */
/* ------------------------------------------------------------------ */

/* RotaryEmbedding::new, qwen3_next.rs:878-904. */
int orc_rope_tables(int n_rot, int64_t max_pos, double theta, float *cos_out, float *sin_out) {
  if (n_rot <= 0 || (n_rot & 1) || max_pos < 0) return ORC_ERR_ARG;
  const int half = n_rot / 2;
  float *inv = (float *)malloc((size_t)half * sizeof(float));
  for (int i = 0; i < half; ++i) {
    /* (0..n_rot).step_by(2): exponent (2i as f64) / (n_rot as f64) */
    const float p = (float)pow(theta, (double)(2 * i) / (double)n_rot);
    inv[i] = 1.0f / p;
  }
  for (int64_t t = 0; t < max_pos; ++t)
    for (int i = 0; i < half; ++i) {
      const float f = (float)t * inv[i]; /* t.matmul(inv_freq): one product */
      cos_out[(size_t)t * half + i] = cosf(f);
      sin_out[(size_t)t * half + i] = sinf(f);
    }
  free(inv);
  return ORC_OK;
}

/* candle_nn::ops::rms_norm (CPU): qwen3_next.rs:2369 (q_norm), 2389 (k_norm). */
void orc_rms_norm(const float *x, const float *alpha, float eps, size_t rows, int d, float *y) {
  for (size_t r = 0; r < rows; ++r) {
    const float *s = x + r * (size_t)d;
    float *o = y + r * (size_t)d;
    float sum2 = -0.0f; /* Sum for f32 folds from -0.0; same result for any x here */
    for (int e = 0; e < d; ++e) sum2 += s[e] * s[e];
    const float m = sqrtf(sum2 / (float)d + eps);
    for (int e = 0; e < d; ++e) o[e] = s[e] / m * alpha[e];
  }
}

/* candle_nn::rotary_emb::rope on x[.., :n_rot] (RotaryEmbedding::apply, qwen3_next.rs:919-939). */
int orc_rope_rows(float *x, size_t rows, int d, int n_rot, const int64_t *pos,
                  const float *cos_tab, const float *sin_tab) {
  if (n_rot <= 0 || (n_rot & 1) || n_rot > d) return ORC_ERR_ARG;
  const int half = n_rot / 2;
  for (size_t r = 0; r < rows; ++r) {
    float *v = x + r * (size_t)d;
    const float *c = cos_tab + (size_t)pos[r] * half, *s = sin_tab + (size_t)pos[r] * half;
    for (int i = 0; i < half; ++i) {
      const float a = v[i], b = v[i + half];
      v[i] = a * c[i] - b * s[i];
      v[i + half] = a * s[i] + b * c[i];
    }
  }
  return ORC_OK;
}

static int prep_rows(const float *x, int batch, int l, int heads, int d, const float *alpha,
                     float eps, int n_rot, const float *cos_tab, const float *sin_tab,
                     int64_t offset, float *out) {
  const size_t rows = (size_t)batch * l * heads;
  orc_rms_norm(x, alpha, eps, rows, d, out);
  int64_t *pos = (int64_t *)malloc((rows + 1) * sizeof(int64_t));
  for (size_t r = 0; r < rows; ++r) pos[r] = offset + (int64_t)((r / (size_t)heads) % (size_t)l);
  const int rc = orc_rope_rows(out, rows, d, n_rot, pos, cos_tab, sin_tab);
  free(pos);
  return rc;
}

/* FullAttention::forward, qwen3_next.rs:2369 (q_norm), 2389 (k_norm), 2399 (rope). */
int orc_qk_prep(const float *q, const float *k, int batch, int l, int n_heads, int n_kv_heads,
                int d, const float *q_alpha, const float *k_alpha, float eps, int n_rot,
                const float *cos_tab, const float *sin_tab, int64_t offset, float *q_out,
                float *k_out) {
  if (batch < 0 || l < 0 || d <= 0 || offset < 0) return ORC_ERR_ARG;
  if (q != NULL) {
    const int rc = prep_rows(q, batch, l, n_heads, d, q_alpha, eps, n_rot, cos_tab, sin_tab,
                             offset, q_out);
    if (rc != ORC_OK) return rc;
  }
  if (k != NULL)
    return prep_rows(k, batch, l, n_kv_heads, d, k_alpha, eps, n_rot, cos_tab, sin_tab,
                     offset, k_out);
  return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* Gated-DeltaNet autoregressive step (ops.rs:391-403, qwen3_next.rs:3392-3470) */
/* ------------------------------------------------------------------ */

void orc_deltanet_step(const float *q, const float *k, const float *v, const float *gate,
                       const float *beta, float *state, float *gate_offset, float *out,
                       int batch, int heads, int d, float scale, float eps) {
  float *qn = (float *)malloc(sizeof(float) * (size_t)d);
  float *kn = (float *)malloc(sizeof(float) * (size_t)d);
  for (int b = 0; b < batch; ++b)
    for (int h = 0; h < heads; ++h) {
      const size_t hb = (size_t)b * heads + h;
      const float *qh = q + hb * d, *kh = k + hb * d, *vh = v + hb * d;
      float *S = state + hb * (size_t)d * d;
      float sq = 0.0f, sk = 0.0f;
      for (int j = 0; j < d; ++j) {
        sq += qh[j] * qh[j];
        sk += kh[j] * kh[j];
      }
      const float iq = 1.0f / sqrtf(sq + eps), ik = 1.0f / sqrtf(sk + eps);
      for (int j = 0; j < d; ++j) {
        qn[j] = qh[j] * iq * scale;
        kn[j] = kh[j] * ik;
      }
      const float alpha = expf(gate[hb]);
      const float bsig = 1.0f / (1.0f + expf(-beta[hb]));
      for (int i = 0; i < d; ++i) {
        float *row = S + (size_t)i * d;
        float u = 0.0f;
        for (int j = 0; j < d; ++j) {
          row[j] = row[j] * alpha;
          u += row[j] * kn[j];
        }
        const float di = (vh[i] - u) * bsig;
        float o = 0.0f;
        for (int j = 0; j < d; ++j) {
          row[j] = row[j] + kn[j] * di;
          o += row[j] * qn[j];
        }
        out[hb * d + i] = o;
      }
      if (gate_offset) gate_offset[hb] = gate_offset[hb] + gate[hb];
    }
  free(qn);
  free(kn);
}

/* ------------------------------------------------------------------ */
/* Gated output projection with Q4K weights (qwen3_next.rs:2657-2680)  */
/* ------------------------------------------------------------------ */

size_t orc_weight_row_bytes(int w_type, int in_dim) {
  switch (w_type) {
    case ORC_W_Q8_0: return (size_t)(in_dim / 32) * 34;
    case ORC_W_Q4K: return (size_t)(in_dim / 256) * 144;
    case ORC_W_Q5K: return (size_t)(in_dim / 256) * 176;
    case ORC_W_Q6K: return (size_t)(in_dim / 256) * 210;
    default: return 0;
  }
}

int orc_gated_oproj(const float *attn, const float *gate, const uint8_t *w, int w_type,
                    float *out, int batch, int in_dim, int out_dim) {
  const size_t row_bytes = orc_weight_row_bytes(w_type, in_dim);
  const int blk = w_type == ORC_W_Q8_0 ? 32 : 256;
  if (row_bytes == 0 || in_dim <= 0 || in_dim % blk != 0 || batch < 0 || out_dim < 0)
    return ORC_ERR_ARG;
  float *y = (float *)malloc(sizeof(float) * (size_t)in_dim);
  float *row = (float *)malloc(sizeof(float) * (size_t)in_dim);
  for (int b = 0; b < batch; ++b) {
    const float *x = attn + (size_t)b * in_dim;
    for (int i = 0; i < in_dim; ++i)
      y[i] = gate ? x[i] * (1.0f / (1.0f + expf(-gate[(size_t)b * in_dim + i]))) : x[i];
    for (int o = 0; o < out_dim; ++o) {
      const uint8_t *wr = w + (size_t)o * row_bytes;
      switch (w_type) {
        case ORC_W_Q8_0: orc_q8_0_dequantize(wr, row, (size_t)in_dim); break;
        case ORC_W_Q4K: orc_q4k_dequantize(wr, row, (size_t)in_dim); break;
        case ORC_W_Q5K: orc_q5k_dequantize(wr, row, (size_t)in_dim); break;
        default: orc_q6k_dequantize(wr, row, (size_t)in_dim); break;
      }
      float acc = 0.0f;
      for (int i = 0; i < in_dim; ++i) acc += row[i] * y[i];
      out[(size_t)b * out_dim + o] = acc;
    }
  }
  free(y);
  free(row);
  return ORC_OK;
}

void orc_gated_oproj_q4k(const float *attn, const float *gate, const uint8_t *w, float *out,
                         int batch, int in_dim, int out_dim) {
  (void)orc_gated_oproj(attn, gate, w, ORC_W_Q4K, out, batch, in_dim, out_dim);
}
