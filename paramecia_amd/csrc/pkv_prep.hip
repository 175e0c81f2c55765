// q/k preparation fused into quantize-on-append.
//
// Reference: FullAttention::forward (paramecia-model/src/qwen3_next.rs:2369-2442) runs,
// per layer and step: q_norm on q [b, l, H, d] (candle_nn::ops::rms_norm), k_norm on k
// [b, l, Hkv, d], the transposes to [b, h, l, d], RotaryEmbedding::apply on the first
// n_rot dims (qwen3_next.rs:906-940, candle_nn::rotary_emb::rope, half-split pairs
// (i, i + n_rot/2)) at positions offset + t, and only then append_quantized. Each step
// is its own pass over the rows. Here one launch takes the projection outputs as they
// are ([b, l, h, d]), and finishes each row in one place: a q row (one wave) is normalised
// and rotated into q_out; a K row (one workgroup) is normalised, rotated and encoded into
// the cache; a V row (one workgroup) is encoded. The encoders are the append path's own (Q4K lane quantizer, Q8_0, f16,
// bf16), so the cache bytes equal those of pkv_append on the prepared rows.
//
// Bit-exactness: candle's CPU rms_norm sums x*x sequentially in f32 and computes
// x / sqrt(sum / d + eps) * alpha; rope computes x1*cos - x2*sin and x1*sin + x2*cos
// with every product rounded. Contraction is off for this file, division and sqrt are
// IEEE (hipcc's defaults), and one lane replays the sum in element order.
#pragma clang fp contract(off)

#include "pkv_internal.hpp"
#include "pkv_scalar.hpp"
#include "pkv_q4k_lanes.hpp"
#include "pkv_prep_common.hpp"

namespace pkv {
namespace {

constexpr int kPrepThreads = 256;  // a K/V row: thread tid owns elements tid, tid + 256
constexpr int kQRowsPerWG = 4;     // q rows of d <= 256: one wave each, 4 elements a lane

struct PrepSmem {
  union {
    struct {
      __attribute__((aligned(16))) float row[512];  // squares, then the normalised row
      float m;
      Q4kScratch q4;
    } kv;
    struct {
      __attribute__((aligned(16))) float row[kQRowsPerWG][256];
      float m[kQRowsPerWG];
    } q;
  };
};

// One wave normalises and rotates a q row of d <= 256 values (lane l: elements 4l..4l+3,
// zero past d), with the same arithmetic as prep_row. row: this wave's 256 LDS floats.
__device__ __forceinline__ void prep_row_wave(float (&x)[4], const PrepElem (&pe)[4], int d,
                                              float eps, int n_rot, float *row, float *m,
                                              int lane) {
#pragma clang fp contract(off)
  *reinterpret_cast<float4 *>(row + 4 * lane) =
      float4{x[0] * x[0], x[1] * x[1], x[2] * x[2], x[3] * x[3]};
  __builtin_amdgcn_wave_barrier();
  if (lane == 0) {
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
  __builtin_amdgcn_wave_barrier();
  const float mm = *m;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (4 * lane + i < d) x[i] = x[i] / mm * pe[i].alpha;
  if (n_rot == 0) return;
  *reinterpret_cast<float4 *>(row + 4 * lane) = float4{x[0], x[1], x[2], x[3]};
  __builtin_amdgcn_wave_barrier();
  const int half = n_rot >> 1;
  float r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = 4 * lane + i;
    if (e >= n_rot)
      r[i] = x[i];
    else if (e < half)
      r[i] = x[i] * pe[i].c - row[e + half] * pe[i].s;
    else
      r[i] = row[e - half] * pe[i].s + x[i] * pe[i].c;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = r[i];
}

// Q8_0 (BlockQ8_0::from_float) of element e of a row, 32 lanes per block: the maximum
// of |x| over the block is exact in any order (NaN dropped, as f32::max does).
__device__ __forceinline__ void q8_encode(float x, int e, uint8_t *row) {
  const int32_t key = (x != x) ? 0 : (int32_t)(f2u(x) & 0x7FFFFFFFu);
  const int32_t kmax = halfwave_allreduce(key, [](int32_t p, int32_t q) { return p > q ? p : q; });
  const float amax = u2f((uint32_t)kmax);
  const float d = amax / 127.0f;
  const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
  uint8_t *blk = row + (e >> 5) * 34;
  blk[2 + (e & 31)] = (uint8_t)rs_as_i8(__builtin_roundf(x * id));
  if ((e & 31) == 0) *reinterpret_cast<uint16_t *>(blk) = f32_to_f16(d);
}

// Workgroups [0, q_wgs) prepare q rows (kQRowsPerWG per workgroup when d <= 256, else
// one), then one workgroup per K row, then one per V row. Every global load of a row
// (x, alpha, cos / sin) is issued before the first barrier.
__global__ __launch_bounds__(kPrepThreads) void prep_append_kernel(PrepArgs a, int64_t q_wgs) {
  __shared__ PrepSmem S;
  const int tid = threadIdx.x;
  const int64_t r = blockIdx.x;
  const int d = a.head_dim, n_rot = a.n_rot, half = n_rot >> 1;
  const bool q_by_wave = d <= 256;
  if (r < q_wgs && q_by_wave) {
    const int lane = tid & 63, w = tid >> 6;
    const int64_t i = r * kQRowsPerWG + w;
    if (i >= a.q_rows) return;  // no workgroup barrier on this path
    const int64_t t = (i / a.num_heads) % a.l;
    const int64_t pos = a.t0 + t;
    const float *src = a.q + i * d;
    float x[4];
    PrepElem pe[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int e = 4 * lane + k;
      x[k] = e < d ? src[e] : 0.0f;
      pe[k] = load_prep_elem(a.q_alpha, a.cos_tab + pos * half, a.sin_tab + pos * half, e, d,
                             n_rot);
    }
    prep_row_wave(x, pe, d, a.eps, n_rot, S.q.row[w], &S.q.m[w], lane);
    float *o = a.q_out + i * d;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (4 * lane + k < d) o[4 * lane + k] = x[k];
    return;
  }
  // one row per workgroup from here on
  int kind;  // 0 q (d > 256), 1 K, 2 V
  int64_t i;
  if (r < q_wgs) {
    kind = 0;
    i = r;
  } else if (r < q_wgs + a.kv_rows) {
    kind = 1;
    i = r - q_wgs;
  } else {
    kind = 2;
    i = r - q_wgs - a.kv_rows;
  }
  const int heads = kind == 0 ? a.num_heads : a.kv_heads;
  const int h = (int)(i % heads);
  const int64_t bt = i / heads;  // b * l + t
  const int64_t t = bt % a.l;
  const int b = (int)(bt / a.l);
  const int64_t pos = a.t0 + t;
  const float *src = (kind == 0 ? a.q : kind == 1 ? a.k : a.v) + i * d;
  float x[2] = {tid < d ? src[tid] : 0.0f, tid + 256 < d ? src[tid + 256] : 0.0f};
  if (kind != 2) {
    const float *al = kind == 0 ? a.q_alpha : a.k_alpha;
    const PrepElem pe[2] = {
        load_prep_elem(al, a.cos_tab + pos * half, a.sin_tab + pos * half, tid, d, n_rot),
        load_prep_elem(al, a.cos_tab + pos * half, a.sin_tab + pos * half, tid + 256, d, n_rot)};
    Q4kWorkgroupBarrier bar;
    prep_row<2>(x, pe, d, a.eps, n_rot, S.kv.row, &S.kv.m, tid, bar);
  }
  if (kind == 0) {
    float *o = a.q_out + i * d;
    if (tid < d) o[tid] = x[0];
    if (tid + 256 < d) o[tid + 256] = x[1];
    return;
  }
  uint8_t *row = (kind == 1 ? a.kc : a.vc) + (((a.t0 + t) * a.batch + b) * a.kv_heads + h) * a.bpr;
  if (a.quant == PKV_QUANT_Q4K) {
    q4k_quantize_superblock_lanes(x[0], row, &S.kv.q4, tid);
    if (a.padded > 256) q4k_quantize_superblock_lanes(x[1], row + 144, &S.kv.q4, tid);
  } else if (a.quant == PKV_QUANT_Q8_0) {
    if (tid < a.padded) q8_encode(x[0], tid, row);
    if (tid + 256 < a.padded) q8_encode(x[1], tid + 256, row);
  } else {
    uint16_t *dst = reinterpret_cast<uint16_t *>(row);
    const bool bf = a.quant == PKV_QUANT_BF16;
    if (tid < a.padded) dst[tid] = bf ? f32_to_bf16(x[0]) : f32_to_f16(x[0]);
    if (tid + 256 < a.padded) dst[tid + 256] = bf ? f32_to_bf16(x[1]) : f32_to_f16(x[1]);
  }
}

}  // namespace

int launch_prep_append(const PrepArgs &a, hipStream_t s) {
  if (a.head_dim > 512 || a.padded > 512) return set_error(PKV_ERR_UNSUPPORTED, "head_dim > 512");
  const int64_t q_wgs =
      a.head_dim <= 256 ? (a.q_rows + kQRowsPerWG - 1) / kQRowsPerWG : a.q_rows;
  const int64_t grid = q_wgs + 2 * a.kv_rows;
  if (grid == 0) return PKV_OK;
  if (grid >= (1ll << 31)) return set_error(PKV_ERR_ARG, "too many rows in one append");
  hipLaunchKernelGGL(prep_append_kernel, dim3((unsigned)grid), dim3(kPrepThreads), 0, s, a,
                     q_wgs);
  PKV_HIP(hipGetLastError());
  return PKV_OK;
}

}  // namespace pkv
