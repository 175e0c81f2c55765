// Gated-DeltaNet autoregressive step for gfx950: the fused kernel behind
// paramecia-model/src/ops.rs:391-403 (delta_net_autoregressive_step), as the Qwen3-Next
// linear-attention layers call it once per token (qwen3_next.rs:3392-3470).
//
// Per (batch b, head h), with the state S[i][j] (i: value channel, j: key channel, the
// roles fixed by qwen3_next.rs:3634-3640):
//   qn = q * scale / sqrt(|q|^2 + eps), kn = k / sqrt(|k|^2 + eps)
//   S = S * exp(gate); u_i = S_i . kn; d_i = (v_i - u_i) * sigmoid(beta)
//   S_i = S_i + d_i kn; out_i = S_i . qn; gate_offset += gate
//
// HBM-bound: every state element is read once and written once, in place, with
// nontemporal accesses (the state comes back only after the other 47 layers). A group of
// 16 lanes owns one row S_i (d / 16 consecutive floats per lane, float4 accesses), so a
// row's two dot products are 16-lane DPP reductions and the update needs no exchange
// beyond them. Each group also normalises its head's q and k from the raw vectors (d
// floats each, L2 hits after the first group of the head).
#include <type_traits>

#include "pkv_internal.hpp"

namespace pkv {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
struct DeltaNetArgs {
  const float *q, *k, *v, *gate, *beta;
  float *state, *gate_offset, *out;
  int heads;
  float scale, eps;
};

// Sum over the 16 lanes of a row (every lane receives it): DPP within rows of 16.
__device__ __forceinline__ float row16_sum(float x) {
  auto dpp = [](float v, auto ctrl) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v),
                                                                __builtin_bit_cast(int, v),
                                                                decltype(ctrl)::value, 0xF, 0xF,
                                                                false));
  };
  x += dpp(x, std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]
  x += dpp(x, std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]
  x += dpp(x, std::integral_constant<int, 0x141>{});  // row_half_mirror
  x += dpp(x, std::integral_constant<int, 0x140>{});  // row_mirror
  return x;
}

template <int kEpl>  // floats per lane: head_dim / 16
__global__ __launch_bounds__(256) void deltanet_step_kernel(DeltaNetArgs a) {
  constexpr int kD = 16 * kEpl, kV4 = kEpl / 4;
  const int lane = threadIdx.x & 15;
  const int row = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int64_t hb = (int64_t)blockIdx.z * a.heads + blockIdx.y;
  const float4 *q4 = reinterpret_cast<const float4 *>(a.q + hb * kD) + kV4 * lane;
  const float4 *k4 = reinterpret_cast<const float4 *>(a.k + hb * kD) + kV4 * lane;
  float4 *s4 = reinterpret_cast<float4 *>(a.state + (hb * kD + row) * kD) + kV4 * lane;
  float qv[kEpl], kv[kEpl], sv[kEpl];
#pragma unroll
  for (int c = 0; c < kV4; ++c) {
    const float4 x = q4[c], y = k4[c], z = __builtin_bit_cast(float4, __builtin_nontemporal_load(reinterpret_cast<const v4f *>(s4) + c));
    qv[4 * c] = x.x; qv[4 * c + 1] = x.y; qv[4 * c + 2] = x.z; qv[4 * c + 3] = x.w;
    kv[4 * c] = y.x; kv[4 * c + 1] = y.y; kv[4 * c + 2] = y.z; kv[4 * c + 3] = y.w;
    sv[4 * c] = z.x; sv[4 * c + 1] = z.y; sv[4 * c + 2] = z.z; sv[4 * c + 3] = z.w;
  }
  const float vi = a.v[hb * kD + row], g = a.gate[hb], bt = a.beta[hb];
  float sq = 0.0f, sk = 0.0f;
#pragma unroll
  for (int e = 0; e < kEpl; ++e) {
    sq = fmaf(qv[e], qv[e], sq);
    sk = fmaf(kv[e], kv[e], sk);
  }
  sq = row16_sum(sq);
  sk = row16_sum(sk);
  const float iq = a.scale / __builtin_sqrtf(sq + a.eps), ik = 1.0f / __builtin_sqrtf(sk + a.eps);
  const float alpha = expf(g), bsig = 1.0f / (1.0f + expf(-bt));
  float u = 0.0f;
#pragma unroll
  for (int e = 0; e < kEpl; ++e) {
    kv[e] *= ik;
    sv[e] *= alpha;
    u = fmaf(sv[e], kv[e], u);
  }
  u = row16_sum(u);
  const float di = (vi - u) * bsig;
  float o = 0.0f;
#pragma unroll
  for (int e = 0; e < kEpl; ++e) {
    sv[e] = fmaf(kv[e], di, sv[e]);
    o = fmaf(sv[e], qv[e] * iq, o);
  }
#pragma unroll
  for (int c = 0; c < kV4; ++c)
    __builtin_nontemporal_store(v4f{sv[4 * c], sv[4 * c + 1], sv[4 * c + 2], sv[4 * c + 3]}, reinterpret_cast<v4f *>(s4) + c);
  o = row16_sum(o);
  if (lane == 0) a.out[hb * kD + row] = o;
  if (a.gate_offset != nullptr && blockIdx.x == 0 && threadIdx.x == 0)
    a.gate_offset[hb] = a.gate_offset[hb] + g;
}

}  // namespace

int launch_deltanet_step(const float *q, const float *k, const float *v, const float *gate,
                         const float *beta, float *state, float *gate_offset, float *out,
                         int batch, int heads, int head_dim, float scale, float eps,
                         hipStream_t s) {
  for (const void *p : {(const void *)q, (const void *)k, (const void *)state})
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
      return set_error(PKV_ERR_ARG, "q, k and state must be 16-byte aligned");
  if (heads > 65535 || batch > 65535) return set_error(PKV_ERR_ARG, "heads and batch must be <= 65535");
  DeltaNetArgs a{q, k, v, gate, beta, state, gate_offset, out, heads, scale, eps};
  const dim3 grid((unsigned)(head_dim / 16), (unsigned)heads, (unsigned)batch);
  switch (head_dim) {
    case 64: hipLaunchKernelGGL(deltanet_step_kernel<4>, grid, dim3(256), 0, s, a); break;
    case 128: hipLaunchKernelGGL(deltanet_step_kernel<8>, grid, dim3(256), 0, s, a); break;
    case 256: hipLaunchKernelGGL(deltanet_step_kernel<16>, grid, dim3(256), 0, s, a); break;
    default:
      return set_error(PKV_ERR_UNSUPPORTED, "delta net step: head_dim must be 64, 128 or 256");
  }
  PKV_HIP(hipGetLastError());
  return PKV_OK;
}

}  // namespace pkv
