// q/k preparation fused into quantize-on-append.
//
// Reference: FullAttention::forward (paramecia-model/src/qwen3_next.rs:2369-2442) runs,
// per layer and step: q_norm on q [b, l, H, d] (candle_nn::ops::rms_norm), k_norm on k
// [b, l, Hkv, d], the transposes to [b, h, l, d], RotaryEmbedding::apply on the first
// n_rot dims (qwen3_next.rs:906-940, candle_nn::rotary_emb::rope, half-split pairs
// (i, i + n_rot/2)) at positions offset + t, and only then append_quantized. Each step
// is its own pass over the rows. Here one launch takes the projection outputs as they
// are ([b, l, h, d]), and each workgroup finishes one row: a q row is normalised and
// rotated into q_out; a K row is normalised, rotated and encoded into the cache; a V row
// is encoded. The encoders are the append path's own (Q4K lane quantizer, Q8_0, f16,
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

namespace pkv {
namespace {

constexpr int kPrepThreads = 256;  // thread tid owns elements tid and tid + 256

struct PrepSmem {
  float row[512];  // squares, then the normalised row (rope partners)
  float m;
  Q4kScratch q4;
};

// Normalise (alpha != null) and rotate (n_rot > 0) the row held as (x0, x1) by the
// workgroup: x0 = element tid, x1 = element tid + 256, zero past d.
__device__ __forceinline__ void prep_row(float &x0, float &x1, const PrepArgs &a,
                                         const float *alpha, int64_t pos, PrepSmem &S,
                                         int tid) {
  const int d = a.head_dim;
  S.row[tid] = x0 * x0;
  S.row[tid + 256] = x1 * x1;
  __syncthreads();
  if (tid == 0) {
    // sum2 = sequential f32 sum of x*x in element order (Rust's Sum folds from -0.0)
    float sum2 = -0.0f;
    const float4 *r4 = reinterpret_cast<const float4 *>(S.row);
    int e = 0;
    for (; e + 4 <= d; e += 4) {
      const float4 t = r4[e >> 2];
      sum2 += t.x;
      sum2 += t.y;
      sum2 += t.z;
      sum2 += t.w;
    }
    for (; e < d; ++e) sum2 += S.row[e];
    S.m = __builtin_sqrtf(sum2 / (float)d + a.eps);
  }
  __syncthreads();
  const float m = S.m;
  if (tid < d) x0 = x0 / m * alpha[tid];
  if (tid + 256 < d) x1 = x1 / m * alpha[tid + 256];
  const int n_rot = a.n_rot;
  if (n_rot == 0) return;
  S.row[tid] = x0;
  S.row[tid + 256] = x1;
  __syncthreads();
  const int half = n_rot >> 1;
  const float *cs = a.cos_tab + pos * half, *sn = a.sin_tab + pos * half;
  auto rot = [&](float y, int e) {
    if (e >= n_rot) return y;
    if (e < half) return y * cs[e] - S.row[e + half] * sn[e];
    return S.row[e - half] * sn[e - half] + y * cs[e - half];
  };
  const float r0 = rot(x0, tid), r1 = rot(x1, tid + 256);
  x0 = r0;
  x1 = r1;
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

__global__ __launch_bounds__(kPrepThreads) void prep_append_kernel(PrepArgs a) {
  __shared__ PrepSmem S;
  const int tid = threadIdx.x;
  const int64_t r = blockIdx.x;
  const int d = a.head_dim;
  int kind;  // 0 q, 1 K, 2 V
  int64_t i;
  if (r < a.q_rows) {
    kind = 0;
    i = r;
  } else if (r < a.q_rows + a.kv_rows) {
    kind = 1;
    i = r - a.q_rows;
  } else {
    kind = 2;
    i = r - a.q_rows - a.kv_rows;
  }
  const int heads = kind == 0 ? a.num_heads : a.kv_heads;
  const int h = (int)(i % heads);
  const int64_t bt = i / heads;  // b * l + t
  const int64_t t = bt % a.l;
  const int b = (int)(bt / a.l);
  const float *src = (kind == 0 ? a.q : kind == 1 ? a.k : a.v) + i * d;
  float x0 = tid < d ? src[tid] : 0.0f;
  float x1 = tid + 256 < d ? src[tid + 256] : 0.0f;
  const int64_t pos = a.t0 + t;
  if (kind != 2) prep_row(x0, x1, a, kind == 0 ? a.q_alpha : a.k_alpha, pos, S, tid);
  if (kind == 0) {
    float *o = a.q_out + i * d;
    if (tid < d) o[tid] = x0;
    if (tid + 256 < d) o[tid + 256] = x1;
    return;
  }
  uint8_t *row = (kind == 1 ? a.kc : a.vc) + (((a.t0 + t) * a.batch + b) * a.kv_heads + h) * a.bpr;
  if (a.quant == PKV_QUANT_Q4K) {
    q4k_quantize_superblock_lanes(x0, row, &S.q4, tid);
    if (a.padded > 256) q4k_quantize_superblock_lanes(x1, row + 144, &S.q4, tid);
  } else if (a.quant == PKV_QUANT_Q8_0) {
    if (tid < a.padded) q8_encode(x0, tid, row);
    if (tid + 256 < a.padded) q8_encode(x1, tid + 256, row);
  } else {
    uint16_t *dst = reinterpret_cast<uint16_t *>(row);
    const bool bf = a.quant == PKV_QUANT_BF16;
    if (tid < a.padded) dst[tid] = bf ? f32_to_bf16(x0) : f32_to_f16(x0);
    if (tid + 256 < a.padded) dst[tid + 256] = bf ? f32_to_bf16(x1) : f32_to_f16(x1);
  }
}

}  // namespace

int launch_prep_append(const PrepArgs &a, hipStream_t s) {
  if (a.head_dim > 512 || a.padded > 512) return set_error(PKV_ERR_UNSUPPORTED, "head_dim > 512");
  const int64_t grid = a.q_rows + 2 * a.kv_rows;
  if (grid == 0) return PKV_OK;
  if (grid >= (1ll << 31)) return set_error(PKV_ERR_ARG, "too many rows in one append");
  hipLaunchKernelGGL(prep_append_kernel, dim3((unsigned)grid), dim3(kPrepThreads), 0, s, a);
  PKV_HIP(hipGetLastError());
  return PKV_OK;
}

}  // namespace pkv
