// Attention over the packed KV rows: generic split-K path (every storage format,
// head_dim <= 512, any GQA ratio up to 16) and the split combine.
//
// Semantics follow the reference CPU SDPA (paramecia-model/src/qwen3_next.rs:2580-2605):
// query head g reads KV head g / (H / Hkv) (repeat_kv, utils.rs:71-83), scores are
// q.k * scale, masked keys (j > i + q_offset when causal) are excluded, scores are
// clamped to [-100, 100], soft-maxed and applied to V. The reference adds -inf before
// the clamp, so its masked keys keep a weight of exp(-100 - max) < 4e-44 of the
// total; skipping them is far inside the attention tolerance.
#include "pkv_internal.hpp"
#include "pkv_scalar.hpp"

namespace pkv {

// Forward declaration: fast MFMA paths (pkv_attn_mfma.hip). Return PKV_ERR_UNSUPPORTED
// when the shape or format has no specialised kernel.
int launch_attend_mfma(const AttnArgs &a, const float *k_new, const float *v_new,
                       uint8_t *kc, uint8_t *vc, int64_t t_new, Workspace &ws,
                       hipStream_t s);
int launch_append_attend_batched_mfma(int quant, const SeqDesc *seqs, int n, const float *k,
                                      const float *v, const float *q, int num_heads,
                                      int num_kv_heads, int head_dim, float scale, float *out,
                                      Workspace &ws, hipStream_t s);
// Q8_0 decode for the Qwen3-Next shape (pkv_q8_decode.hip).
int launch_attend_q8(const AttnArgs &a, const float *k_new, const float *v_new, uint8_t *kc,
                     uint8_t *vc, int64_t t_new, Workspace &ws, hipStream_t s);
int launch_append_attend_batched_q8(int quant, const SeqDesc *seqs, int n, const float *k,
                                    const float *v, const float *q, int num_heads,
                                    int num_kv_heads, int head_dim, float scale, float *out,
                                    Workspace &ws, hipStream_t s);
// Prefill chunk (l > 1) over Q4K rows of the Qwen3-Next shape (pkv_prefill_mfma.hip).
int launch_prefill_mfma(const AttnArgs &a, Workspace &ws, hipStream_t s);
int launch_prefill_q8_mfma(const AttnArgs &a, Workspace &ws, hipStream_t s);

namespace {

constexpr int kWaves = 4;

struct Partials {
  float *m;  // [splits][rows] running max of clamped scores
  float *l;  // [splits][rows] sum of exp(score - m)
  float *o;  // [splits][rows][head_dim] un-normalised sum of p * v
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// One wave = one split of the keys of one (batch, query, kv head) group.
template <int G, int R>
__global__ __launch_bounds__(kWaves * 64) void generic_partial_kernel(AttnArgs a,
                                                                     int64_t keys_per_wave,
                                                                     int waves_per_group,
                                                                     Partials P) {
  __shared__ float qs[G * R * 64];
  const int gi = blockIdx.y;  // ((b * l) + i) * Hkv + kh
  const int kh = gi % a.num_kv_heads;
  const int i = (gi / a.num_kv_heads) % a.l;
  const int b = gi / (a.num_kv_heads * a.l);
  const int D = a.head_dim;
  for (int x = threadIdx.x; x < G * R * 64; x += blockDim.x) {
    const int g = x / (R * 64), e = x % (R * 64);
    qs[x] = e < D ? a.q[(((int64_t)b * a.l + i) * a.num_heads + kh * G + g) * D + e] : 0.0f;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * kWaves + (threadIdx.x >> 6);
  const int64_t kend = a.causal ? (a.q_offset + i + 1 < a.seq_k ? a.q_offset + i + 1 : a.seq_k)
                                : a.seq_k;
  const int64_t k0 = (int64_t)wave * keys_per_wave;
  const int64_t k1 = k0 + keys_per_wave < kend ? k0 + keys_per_wave : kend;

  float m[G], lsum[G], acc[G][R];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    lsum[g] = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) acc[g][r] = 0.0f;
  }
  const uint8_t *kbase = a.k + b * a.rs.b + kh * a.rs.h;
  const uint8_t *vbase = a.v + b * a.rs.b + kh * a.rs.h;
  for (int64_t j = k0; j < k1; ++j) {
    float kr[R], vr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int e = lane + 64 * r;
      kr[r] = e < D ? decode_elem(a.quant, kbase + j * a.rs.t, e) : 0.0f;
      vr[r] = e < D ? decode_elem(a.quant, vbase + j * a.rs.t, e) : 0.0f;
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float part = 0.0f;
#pragma unroll
      for (int r = 0; r < R; ++r) part += qs[g * R * 64 + lane + 64 * r] * kr[r];
      float s = wave_sum(part) * a.scale;
      s = fminf(fmaxf(s, -100.0f), 100.0f);
      const float mn = fmaxf(m[g], s);
      const float c = __expf(m[g] - mn);
      const float p = __expf(s - mn);
      lsum[g] = lsum[g] * c + p;
#pragma unroll
      for (int r = 0; r < R; ++r) acc[g][r] = acc[g][r] * c + p * vr[r];
      m[g] = mn;
    }
  }
  const int rows = a.batch * a.l * a.num_heads;
  const int64_t split = (int64_t)wave;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int row = ((b * a.l) + i) * a.num_heads + kh * G + g;
    if (lane == 0) {
      P.m[split * rows + row] = m[g];
      P.l[split * rows + row] = lsum[g];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int e = lane + 64 * r;
      if (e < D) P.o[(split * rows + row) * D + e] = acc[g][r];
    }
  }
  (void)waves_per_group;
}

// out[row] = sum_s o_s * e^{m_s - M} / sum_s l_s * e^{m_s - M}
__global__ __launch_bounds__(256) void combine_kernel(Partials P, int splits, int rows, int D,
                                                      float *out) {
  extern __shared__ float w[];  // [splits]
  __shared__ float red[256];
  const int row = blockIdx.x;
  float mx = -INFINITY;
  for (int s = threadIdx.x; s < splits; s += blockDim.x) mx = fmaxf(mx, P.m[(int64_t)s * rows + row]);
  red[threadIdx.x] = mx;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + o]);
    __syncthreads();
  }
  mx = red[0];
  __syncthreads();
  float lsum = 0.0f;
  for (int s = threadIdx.x; s < splits; s += blockDim.x) {
    const float ms = P.m[(int64_t)s * rows + row];
    const float ws = (ms == -INFINITY) ? 0.0f : __expf(ms - mx);
    w[s] = ws;
    lsum += ws * P.l[(int64_t)s * rows + row];
  }
  red[threadIdx.x] = lsum;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  const float inv = red[0] > 0.0f ? 1.0f / red[0] : 0.0f;
  for (int e = threadIdx.x; e < D; e += blockDim.x) {
    float acc = 0.0f;
    for (int s = 0; s < splits; ++s) acc += w[s] * P.o[((int64_t)s * rows + row) * D + e];
    out[(int64_t)row * D + e] = acc * inv;
  }
}

template <int G>
int launch_generic_g(const AttnArgs &a, int R, dim3 grid, int64_t kpw, int wpg, Partials P,
                     hipStream_t s) {
  switch (R) {
    case 1: hipLaunchKernelGGL((generic_partial_kernel<G, 1>), grid, dim3(kWaves * 64), 0, s, a, kpw, wpg, P); break;
    case 2: hipLaunchKernelGGL((generic_partial_kernel<G, 2>), grid, dim3(kWaves * 64), 0, s, a, kpw, wpg, P); break;
    case 4: hipLaunchKernelGGL((generic_partial_kernel<G, 4>), grid, dim3(kWaves * 64), 0, s, a, kpw, wpg, P); break;
    default: hipLaunchKernelGGL((generic_partial_kernel<G, 8>), grid, dim3(kWaves * 64), 0, s, a, kpw, wpg, P); break;
  }
  return PKV_OK;
}

}  // namespace

int launch_attend_generic(const AttnArgs &a, Workspace &ws, hipStream_t s) {
  const int G = a.num_heads / a.num_kv_heads;
  const int R = a.head_dim <= 64 ? 1 : a.head_dim <= 128 ? 2 : a.head_dim <= 256 ? 4 : 8;
  const int groups = a.batch * a.l * a.num_kv_heads;
  // Enough waves to fill the GPU, at least 16 keys per wave.
  int64_t want = (16384 + groups - 1) / groups;
  if (want > 4096) want = 4096;  // combine keeps one weight per split in LDS
  int64_t max_waves = (a.seq_k + 15) / 16;
  int64_t wpg = want < max_waves ? want : max_waves;
  wpg = (wpg + kWaves - 1) / kWaves * kWaves;
  if (wpg < kWaves) wpg = kWaves;
  const int64_t kpw = (a.seq_k + wpg - 1) / wpg;
  const int rows = a.batch * a.l * a.num_heads;
  const size_t need = (size_t)wpg * rows * (2 + (size_t)a.head_dim) * sizeof(float);
  int rc = ws.reserve(need);
  if (rc) return rc;
  Partials P;
  P.m = reinterpret_cast<float *>(ws.ptr);
  P.l = P.m + (size_t)wpg * rows;
  P.o = P.l + (size_t)wpg * rows;
  dim3 grid((unsigned)(wpg / kWaves), (unsigned)groups);
  switch (G) {
    case 1: rc = launch_generic_g<1>(a, R, grid, kpw, (int)wpg, P, s); break;
    case 2: rc = launch_generic_g<2>(a, R, grid, kpw, (int)wpg, P, s); break;
    case 4: rc = launch_generic_g<4>(a, R, grid, kpw, (int)wpg, P, s); break;
    case 8: rc = launch_generic_g<8>(a, R, grid, kpw, (int)wpg, P, s); break;
    case 16: rc = launch_generic_g<16>(a, R, grid, kpw, (int)wpg, P, s); break;
    default: return set_error(PKV_ERR_UNSUPPORTED, "num_heads / num_kv_heads must be 1, 2, 4, 8 or 16");
  }
  if (rc) return rc;
  PKV_HIP(hipGetLastError());
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)rows), dim3(256), wpg * sizeof(float), s, P,
                     (int)wpg, rows, a.head_dim, a.out);
  PKV_HIP(hipGetLastError());
  return PKV_OK;
}

static int check_attn(const AttnArgs &a) {
  if (a.num_kv_heads <= 0 || a.num_heads % a.num_kv_heads != 0)
    return set_error(PKV_ERR_ARG, "num_heads must be a multiple of num_kv_heads");
  if (a.head_dim <= 0 || a.head_dim > 512)
    return set_error(PKV_ERR_UNSUPPORTED, "head_dim must be in [1, 512]");
  if (a.l <= 0 || a.batch <= 0) return set_error(PKV_ERR_ARG, "batch and l must be positive");
  if (a.seq_k <= 0) return set_error(PKV_ERR_EMPTY, "Cannot attend over an empty cache");
  if (a.q_offset < 0) return set_error(PKV_ERR_ARG, "q_offset must be >= 0");
  return PKV_OK;
}

int launch_attend(const AttnArgs &a, Workspace &ws, hipStream_t s) {
  int rc = check_attn(a);
  if (rc) return rc;
  rc = launch_attend_mfma(a, nullptr, nullptr, nullptr, nullptr, -1, ws, s);
  if (rc != PKV_ERR_UNSUPPORTED) return rc;
  rc = launch_attend_q8(a, nullptr, nullptr, nullptr, nullptr, -1, ws, s);
  if (rc != PKV_ERR_UNSUPPORTED) return rc;
  rc = launch_prefill_mfma(a, ws, s);
  if (rc != PKV_ERR_UNSUPPORTED) return rc;
  rc = launch_prefill_q8_mfma(a, ws, s);
  if (rc != PKV_ERR_UNSUPPORTED) return rc;
  return launch_attend_generic(a, ws, s);
}

int launch_append_attend(const AttnArgs &a, const float *k_new, const float *v_new,
                         uint8_t *kc, uint8_t *vc, int64_t t_new, Workspace &ws,
                         hipStream_t s) {
  int rc = check_attn(a);
  if (rc) return rc;
  rc = launch_attend_mfma(a, k_new, v_new, kc, vc, t_new, ws, s);
  if (rc != PKV_ERR_UNSUPPORTED) return rc;
  rc = launch_attend_q8(a, k_new, v_new, kc, vc, t_new, ws, s);
  if (rc != PKV_ERR_UNSUPPORTED) return rc;
  rc = launch_append(a.quant, k_new, v_new, kc, vc, a.batch, a.num_kv_heads, a.head_dim, 1,
                     t_new, s);
  if (rc) return rc;
  return launch_attend_generic(a, ws, s);
}

int launch_append_attend_batched(int quant, const SeqDesc *seqs, int n, const float *k,
                                 const float *v, const float *q, int num_heads,
                                 int num_kv_heads, int head_dim, float scale, float *out,
                                 Workspace &ws, hipStream_t s) {
  // one launch for every sequence when an MFMA kernel covers the shape
  const int rc0 = launch_append_attend_batched_mfma(quant, seqs, n, k, v, q, num_heads,
                                                    num_kv_heads, head_dim, scale, out, ws, s);
  if (rc0 != PKV_ERR_UNSUPPORTED) return rc0;
  const int rc1 = launch_append_attend_batched_q8(quant, seqs, n, k, v, q, num_heads,
                                                  num_kv_heads, head_dim, scale, out, ws, s);
  if (rc1 != PKV_ERR_UNSUPPORTED) return rc1;
  const size_t kv_stride = (size_t)num_kv_heads * head_dim;
  const size_t q_stride = (size_t)num_heads * head_dim;
  const int64_t bpr = (int64_t)row_bytes(quant, head_dim);
  for (int i = 0; i < n; ++i) {
    AttnArgs a;
    a.quant = quant;
    a.q = q + i * q_stride;
    a.k = seqs[i].k;
    a.v = seqs[i].v;
    a.rs = {num_kv_heads * bpr, num_kv_heads * bpr, bpr};
    a.scale = scale;
    a.batch = 1;
    a.num_heads = num_heads;
    a.num_kv_heads = num_kv_heads;
    a.head_dim = head_dim;
    a.l = 1;
    a.seq_k = seqs[i].len;
    a.q_offset = seqs[i].len - 1;
    a.causal = 1;
    a.out = out + i * q_stride;
    int rc = launch_append_attend(a, k + i * kv_stride, v + i * kv_stride, seqs[i].k, seqs[i].v,
                                  seqs[i].len - 1, ws, s);
    if (rc) return rc;
  }
  return PKV_OK;
}

}  // namespace pkv
