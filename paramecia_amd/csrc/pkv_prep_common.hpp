// Row preparation ahead of the cache: q_norm / k_norm (candle_nn::ops::rms_norm) and the
// partial rope (candle_nn::rotary_emb::rope on the first n_rot values, half-split pairs
// (i, i + n_rot/2)), as FullAttention::forward applies them (paramecia-model/src/
// qwen3_next.rs:2369-2399, RotaryEmbedding::apply :906-940). Shared by the prep-append
// kernel and the fused decode kernel. Include-only; every a*b+c rounds twice.
//
// candle's CPU rms_norm sums x*x sequentially in f32 and returns x / sqrt(sum / d + eps)
// * alpha; one lane replays the sum in element order, so the result is bit-exact.
#pragma once
#include "pkv_scalar.hpp"

namespace pkv {

// What the thread owning element e of a row needs besides x: alpha[e], and for e < n_rot
// the cos and sin of rope index e mod (n_rot / 2) at the row's position.
struct PrepElem {
  float alpha, c, s;
};

__device__ __forceinline__ PrepElem load_prep_elem(const float *alpha, const float *cos_row,
                                                   const float *sin_row, int e, int d,
                                                   int n_rot) {
  PrepElem p{1.0f, 1.0f, 0.0f};
  if (e < d) p.alpha = alpha[e];
  if (e < n_rot) {
    const int half = n_rot >> 1;
    const int i = e < half ? e : e - half;
    p.c = cos_row[i];
    p.s = sin_row[i];
  }
  return p;
}

// Normalise and rotate one row held by 256 threads: x[j] is element tid + 256 j (zero
// past d). `row` is LDS of 256 N floats (16-byte aligned), `m` one LDS float; `bar`
// synchronises the 256 threads (three times). The caller synchronises again before it
// rewrites `row`.
template <int N, typename Bar>
__device__ __forceinline__ void prep_row(float (&x)[N], const PrepElem (&pe)[N], int d,
                                         float eps, int n_rot, float *row, float *m, int tid,
                                         Bar &bar) {
#pragma clang fp contract(off)
#pragma unroll
  for (int j = 0; j < N; ++j) row[tid + 256 * j] = x[j] * x[j];
  bar();
  if (tid == 0) {
    // Rust's f32 Sum folds from -0.0, in element order
    float sum2 = -0.0f;
    const float4 *r4 = reinterpret_cast<const float4 *>(row);
    int e = 0;
    for (; e + 4 <= d; e += 4) {
      const float4 t = r4[e >> 2];
      sum2 += t.x;
      sum2 += t.y;
      sum2 += t.z;
      sum2 += t.w;
    }
    for (; e < d; ++e) sum2 += row[e];
    *m = __builtin_sqrtf(sum2 / (float)d + eps);
  }
  bar();
  const float mm = *m;
#pragma unroll
  for (int j = 0; j < N; ++j)
    if (tid + 256 * j < d) x[j] = x[j] / mm * pe[j].alpha;
  if (n_rot == 0) return;
#pragma unroll
  for (int j = 0; j < N; ++j) row[tid + 256 * j] = x[j];
  bar();
  const int half = n_rot >> 1;
  float r[N];
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const int e = tid + 256 * j;
    if (e >= n_rot)
      r[j] = x[j];
    else if (e < half)
      r[j] = x[j] * pe[j].c - row[e + half] * pe[j].s;
    else
      r[j] = row[e - half] * pe[j].s + x[j] * pe[j].c;
  }
#pragma unroll
  for (int j = 0; j < N; ++j) x[j] = r[j];
}

}  // namespace pkv
