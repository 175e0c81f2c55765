// Gated output projection of a full-attention layer with Q4K weights, gfx950: the step
// after the attention (paramecia-model/src/qwen3_next.rs:2657-2680): the attention output
// times sigmoid(gate), then self.wo, a GGUF QMatMul (models/with_tracing.rs:253-300,
// base path without custom scales or LoRA).
//
//   out[b][o] = sum_i W[o][i] * attn[b][i] * sigmoid(gate[b][i])
//
// W is out_dim rows of in_dim / 256 Q4K superblocks (144 B each: f16 d, f16 dmin, 12 B
// of 6-bit scale / min codes, 128 B of nibbles), the GGUF layout. Weight streaming is
// the cost (HBM; latency at batch 1): a workgroup of 4 waves owns 4 output rows (one per
// wave: more workgroups in flight, for one or two tokens) or 8 (two per wave: the gated
// input staged once for more rows, from four tokens on). Its threads first write the gated input row into LDS (each input is gated once
// per workgroup); lane l of a wave then takes 64-element chunk l % 4 of superblock l / 4
// (and further chunks in steps of 64 for wider inputs): the chunk's 32 nibble bytes, its
// two sub-block scales and mins, and a wave reduction give the row's dot product. Each
// token of a batch has its own workgroups (grid y); those of one row group share an XCD
// (same x), so the weights come from HBM once and from that XCD's L2 after.
#include <type_traits>

#include "pkv_internal.hpp"
#include "pkv_scalar.hpp"

namespace pkv {
namespace {

constexpr int kOprojWaves = 4;
constexpr int kOprojMaxIn = 8192;  // LDS: one gated input row
// The gated row sits in LDS as 64-float chunks padded to 68 floats: lane l reads chunk l,
// so without the pad every lane of a ds_read_b128 would hit the same banks (256-byte
// stride)
constexpr int kChunkPad = 68;

struct OprojArgs {
  const float *attn, *gate;  // [batch][in_dim]; gate may be null (no gating)
  const uint8_t *w;          // [out_dim][in_dim / 256][144]
  float *out;                // [batch][out_dim]
  int batch, in_dim, out_dim;
};

__device__ __forceinline__ float wave64_sum(float x) {
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
  {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    x = __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
  }
  {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    x = __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
  }
  return x;
}

// 6-bit scale and min codes of sub-block j from the 12 header bytes (get_scale_min_k4)
__device__ __forceinline__ void q4k_scale_min(const uint8_t *s, int j, float &sc, float &m) {
  if (j < 4) {
    sc = (float)(s[j] & 63);
    m = (float)(s[j + 4] & 63);
  } else {
    sc = (float)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
    m = (float)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
  }
}

// sigmoid(g) through v_exp_f32 and v_rcp_f32 (about 1 ulp each; the projection's
// tolerance is 1e-3 relative)
__device__ __forceinline__ float fast_sigmoid(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f));
}
// the four bytes of w as floats (the backend selects v_cvt_f32_ubyte0..3)
__device__ __forceinline__ void bytes_to_f32(uint32_t w, float *f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) f[i] = (float)((w >> (8 * i)) & 0xFFu);
}

// kChunks 64-element chunks per lane (in_dim / 4096), kOprojRowsPerWave output rows per wave
template <int kChunks, int kOprojRowsPerWave>
__global__ __launch_bounds__(256) void oproj_q4k_kernel(OprojArgs a) {
  __shared__ __attribute__((aligned(16))) float xs[kOprojMaxIn / 64 * kChunkPad];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nsb = a.in_dim >> 8;
  const int row0 = (blockIdx.x * kOprojWaves + wave) * kOprojRowsPerWave;
  const int b = blockIdx.y;
  // the inputs are read before the weights: their loads (L2 hits after the first
  // workgroups) then need not wait behind the weight stream
  constexpr int kIn4 = kChunks * 4;  // float4 of the input row per thread (in_dim / 1024)
  float4 x0[kIn4], g0[kIn4];
#pragma unroll
  for (int k = 0; k < kIn4; ++k) {
    x0[k] = reinterpret_cast<const float4 *>(a.attn + (int64_t)b * a.in_dim)[tid + 256 * k];
    g0[k] = a.gate != nullptr
                ? reinterpret_cast<const float4 *>(a.gate + (int64_t)b * a.in_dim)[tid + 256 * k]
                : float4{0.f, 0.f, 0.f, 0.f};
  }
  // this lane's weights for each of its rows and chunks: the superblock header and the
  // chunk's 32 nibble bytes, decoded only after the input is staged (so that the
  // staging does not wait for the weight stream)
  uint4 hdr[kOprojRowsPerWave][kChunks], nib[kOprojRowsPerWave][kChunks][2];
#pragma unroll
  for (int r = 0; r < kOprojRowsPerWave; ++r)
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch) {
      const int c = 64 * ch + lane, sb = c >> 2, cc = c & 3;
      const int row = row0 + r < a.out_dim ? row0 + r : a.out_dim - 1;
      const uint8_t *blk = a.w + ((int64_t)row * nsb + sb) * 144;
      hdr[r][ch] = *reinterpret_cast<const uint4 *>(blk);
      nib[r][ch][0] = reinterpret_cast<const uint4 *>(blk + 16 + 32 * cc)[0];
      nib[r][ch][1] = reinterpret_cast<const uint4 *>(blk + 16 + 32 * cc)[1];
    }
  {
#pragma unroll
    for (int k = 0; k < kIn4; ++k) {
      float4 x = x0[k];
      if (a.gate != nullptr) {
        x.x *= fast_sigmoid(g0[k].x);
        x.y *= fast_sigmoid(g0[k].y);
        x.z *= fast_sigmoid(g0[k].z);
        x.w *= fast_sigmoid(g0[k].w);
      }
      const int e = 4 * (tid + 256 * k);  // first element of this float4
      *reinterpret_cast<float4 *>(xs + (e >> 6) * kChunkPad + (e & 63)) = x;
    }
    __syncthreads();
    float acc[kOprojRowsPerWave];
#pragma unroll
    for (int r = 0; r < kOprojRowsPerWave; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch) {
      const int c = 64 * ch + lane, cc = c & 3;
      const float *xc = xs + c * kChunkPad;  // chunk c = 4 superblock + cc of the row
      // low nibbles weigh elements 0-31 of the chunk, high nibbles elements 32-63
      float xl[32], xh[32];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float4 l4 = reinterpret_cast<const float4 *>(xc)[i];
        const float4 h4 = reinterpret_cast<const float4 *>(xc + 32)[i];
        xl[4 * i] = l4.x; xl[4 * i + 1] = l4.y; xl[4 * i + 2] = l4.z; xl[4 * i + 3] = l4.w;
        xh[4 * i] = h4.x; xh[4 * i + 1] = h4.y; xh[4 * i + 2] = h4.z; xh[4 * i + 3] = h4.w;
      }
      float sl = 0.0f, sh = 0.0f;
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        sl += xl[i];
        sh += xh[i];
      }
#pragma unroll
      for (int r = 0; r < kOprojRowsPerWave; ++r) {
        const uint32_t w8[8] = {nib[r][ch][0].x, nib[r][ch][0].y, nib[r][ch][0].z, nib[r][ch][0].w,
                                nib[r][ch][1].x, nib[r][ch][1].y, nib[r][ch][1].z, nib[r][ch][1].w};
        float pl[2] = {0.0f, 0.0f}, ph[2] = {0.0f, 0.0f};  // two chains each, for ILP
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          float nl[4], nh[4];
          bytes_to_f32(w8[q] & 0x0F0F0F0Fu, nl);
          bytes_to_f32((w8[q] >> 4) & 0x0F0F0F0Fu, nh);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            pl[q & 1] = fmaf(nl[i], xl[4 * q + i], pl[q & 1]);
            ph[q & 1] = fmaf(nh[i], xh[4 * q + i], ph[q & 1]);
          }
        }
        // the chunk's two sub-blocks: (d * sc, dmin * m) from the superblock header
        const uint4 hd = hdr[r][ch];
        uint8_t sbytes[12];
        const uint32_t hw[3] = {hd.y, hd.z, hd.w};
#pragma unroll
        for (int i = 0; i < 12; ++i) sbytes[i] = (uint8_t)(hw[i >> 2] >> (8 * (i & 3)));
        const float d = f16_to_f32((uint16_t)(hd.x & 0xFFFF)), dmin = f16_to_f32((uint16_t)(hd.x >> 16));
        float sc0, m0, sc1, m1;
        q4k_scale_min(sbytes, 2 * cc, sc0, m0);
        q4k_scale_min(sbytes, 2 * cc + 1, sc1, m1);
        acc[r] += (d * sc0) * (pl[0] + pl[1]) - (dmin * m0) * sl + (d * sc1) * (ph[0] + ph[1]) -
                  (dmin * m1) * sh;
      }
    }
#pragma unroll
    for (int r = 0; r < kOprojRowsPerWave; ++r) {
      const float y = wave64_sum(acc[r]);
      if (lane == 0 && row0 + r < a.out_dim) a.out[(int64_t)b * a.out_dim + row0 + r] = y;
    }
  }
}

}  // namespace

int launch_oproj_q4k(const float *attn, const float *gate, const uint8_t *w, float *out,
                     int batch, int in_dim, int out_dim, hipStream_t s) {
  if (in_dim % 4096 != 0 || in_dim > kOprojMaxIn)
    return set_error(PKV_ERR_UNSUPPORTED, "gated o_proj: in_dim must be 4096 or 8192");
  for (const void *p : {(const void *)attn, (const void *)gate, (const void *)w})
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
      return set_error(PKV_ERR_ARG, "attn, gate and the weights must be 16-byte aligned");
  if (batch > 65535) return set_error(PKV_ERR_ARG, "batch must be <= 65535");
  OprojArgs a{attn, gate, w, out, batch, in_dim, out_dim};
  const int rows_per_wave = batch < 4 ? 1 : 2;
  const int rows_per_wg = kOprojWaves * rows_per_wave;
  const dim3 grid((unsigned)((out_dim + rows_per_wg - 1) / rows_per_wg), (unsigned)batch);
  switch ((in_dim / 4096) * 4 + rows_per_wave) {
    case 5: hipLaunchKernelGGL((oproj_q4k_kernel<1, 1>), grid, dim3(256), 0, s, a); break;
    case 6: hipLaunchKernelGGL((oproj_q4k_kernel<1, 2>), grid, dim3(256), 0, s, a); break;
    case 9: hipLaunchKernelGGL((oproj_q4k_kernel<2, 1>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((oproj_q4k_kernel<2, 2>), grid, dim3(256), 0, s, a); break;
  }
  PKV_HIP(hipGetLastError());
  return PKV_OK;
}

}  // namespace pkv
