// Gated output projection of a full-attention layer, gfx950: the step after the attention
// (paramecia-model/src/qwen3_next.rs:2657-2680): the attention output times
// sigmoid(gate), then self.wo, a GGUF QMatMul (models/with_tracing.rs:253-300, base path
// without custom scales or LoRA).
//
//   out[b][o] = sum_i W[o][i] * attn[b][i] * sigmoid(gate[b][i])
//
// W is out_dim rows of in_dim elements in one GGUF block type (GGML's numbering):
//   Q4K (12) 144 B per 256: f16 d, f16 dmin, 12 B of 6-bit scale / min codes, 128 B nibbles
//   Q5K (13) 176 B per 256: the Q4K header, 32 B of fifth bits, 128 B nibbles
//   Q6K (14) 210 B per 256: 128 B low nibbles, 64 B bit pairs, 16 int8 scales, f16 d
//   Q8_0 (8)  34 B per 32:  f16 d, 32 int8 codes
// This file holds the per-token form (GEMV: weight streaming, HBM- or latency-bound at a
// few tokens). A workgroup of 4 waves owns 4 output rows (one per wave: more workgroups
// in flight, for one to three tokens) or 8 (two per wave: the gated input staged once for
// more rows, from four tokens on). Its threads first write the gated input row into LDS
// (each input is gated once per workgroup). Q4K and Q5K blocks are 16-byte aligned, so
// lane l of a wave loads its weights straight into registers: 64-element chunk l % 4 of
// superblock l / 4 (and further chunks in steps of 64 for wider inputs). Q6K and Q8_0
// blocks are only 2-byte aligned (210 and 34 B), so the workgroup first copies its rows'
// bytes into LDS with aligned 16-byte loads (a row of 4096 or 8192 inputs is a multiple
// of 16 B), and each lane reads its block fields back as aligned dwords shifted by
// v_alignbyte. A wave reduction gives each row's dot product. Each token of a batch has
// its own workgroups (grid y); those of one row group share an XCD (same x), so the
// weights come from HBM once and from that XCD's L2 after.
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

enum : int { kWQ8_0 = 8, kWQ4K = 12, kWQ5K = 13, kWQ6K = 14 };

struct OprojArgs {
  const float *attn, *gate;  // [batch][in_dim]; gate may be null (no gating)
  const uint8_t *w;          // [out_dim][row bytes]
  float *out;                // [batch][out_dim]
  int batch, in_dim, out_dim;
};

__host__ __device__ constexpr int block_elems(int fmt) { return fmt == kWQ8_0 ? 32 : 256; }
__host__ __device__ constexpr int block_bytes(int fmt) {
  return fmt == kWQ8_0 ? 34 : fmt == kWQ4K ? 144 : fmt == kWQ5K ? 176 : 210;
}

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

// 6-bit scale and min codes of sub-block j (get_scale_min_k4) from the 12 header bytes
// held as three little-endian words (header byte i is byte i & 3 of word i >> 2). j may
// differ between lanes: a shift by 8 (j & 3) reads bytes j & 3, 4 + (j & 3) and
// 8 + (j & 3), where an indexed byte array would lower to compare-and-select chains.
__device__ __forceinline__ void q4k_scale_min(uint32_t w0, uint32_t w1, uint32_t w2, int j,
                                              float &sc, float &m) {
  const int sh = 8 * (j & 3);
  const uint32_t b0 = w0 >> sh, b1 = w1 >> sh, b2 = w2 >> sh;
  const uint32_t lo_s = b0 & 63, lo_m = b1 & 63;
  const uint32_t hi_s = (b2 & 0xF) | (((b0 >> 6) & 3) << 4);
  const uint32_t hi_m = ((b2 >> 4) & 0xF) | (((b1 >> 6) & 3) << 4);
  sc = (float)(j < 4 ? lo_s : hi_s);
  m = (float)(j < 4 ? lo_m : hi_m);
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

// Q4K / Q5K. kChunks 64-element chunks per lane (in_dim / 4096), kOprojRowsPerWave output
// rows per wave.
template <int kFmt, int kChunks, int kOprojRowsPerWave>
__global__ __launch_bounds__(256) void oproj_k45_kernel(OprojArgs a) {
  static_assert(kFmt == kWQ4K || kFmt == kWQ5K, "Q4K or Q5K");
  constexpr int kBB = block_bytes(kFmt);
  constexpr int kNibOff = kFmt == kWQ5K ? 48 : 16;  // the nibbles follow the fifth bits
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
  // this lane's weights for each of its rows and chunks: the superblock header, the
  // chunk's 32 nibble bytes and (Q5K) the superblock's 32 bytes of fifth bits, decoded only
  // after the input is staged (so that the staging does not wait for the weight stream)
  constexpr int kHi = kFmt == kWQ5K ? 2 : 1;
  uint4 hdr[kOprojRowsPerWave][kChunks], nib[kOprojRowsPerWave][kChunks][2];
  uint4 fifth[kOprojRowsPerWave][kChunks][kHi];
#pragma unroll
  for (int r = 0; r < kOprojRowsPerWave; ++r)
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch) {
      const int c = 64 * ch + lane, sb = c >> 2, cc = c & 3;
      const int row = row0 + r < a.out_dim ? row0 + r : a.out_dim - 1;
      const uint8_t *blk = a.w + ((int64_t)row * nsb + sb) * kBB;
      hdr[r][ch] = *reinterpret_cast<const uint4 *>(blk);
      nib[r][ch][0] = reinterpret_cast<const uint4 *>(blk + kNibOff + 32 * cc)[0];
      nib[r][ch][1] = reinterpret_cast<const uint4 *>(blk + kNibOff + 32 * cc)[1];
      if constexpr (kFmt == kWQ5K) {
        fifth[r][ch][0] = reinterpret_cast<const uint4 *>(blk + 16)[0];
        fifth[r][ch][1] = reinterpret_cast<const uint4 *>(blk + 16)[1];
      } else {
        fifth[r][ch][0] = uint4{0u, 0u, 0u, 0u};
      }
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
          uint32_t cl = w8[q] & 0x0F0F0F0Fu, chh = (w8[q] >> 4) & 0x0F0F0F0Fu;
          if constexpr (kFmt == kWQ5K) {
            // byte l of the fifth bits carries bit j for element 32 j + l: bits 2 cc and
            // 2 cc + 1 belong to this chunk's two sub-blocks
            const uint4 f4 = fifth[r][ch][q >> 2];
            const uint32_t fw = (q & 3) == 0 ? f4.x : (q & 3) == 1 ? f4.y : (q & 3) == 2 ? f4.z : f4.w;
            cl |= ((fw >> (2 * cc)) & 0x01010101u) << 4;
            chh |= ((fw >> (2 * cc + 1)) & 0x01010101u) << 4;
          }
          float nl[4], nh[4];
          bytes_to_f32(cl, nl);
          bytes_to_f32(chh, nh);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            pl[q & 1] = fmaf(nl[i], xl[4 * q + i], pl[q & 1]);
            ph[q & 1] = fmaf(nh[i], xh[4 * q + i], ph[q & 1]);
          }
        }
        // the chunk's two sub-blocks: (d * sc, dmin * m) from the superblock header
        const uint4 hd = hdr[r][ch];
        const float d = f16_to_f32((uint16_t)(hd.x & 0xFFFF)), dmin = f16_to_f32((uint16_t)(hd.x >> 16));
        float sc0, m0, sc1, m1;
        q4k_scale_min(hd.y, hd.z, hd.w, 2 * cc, sc0, m0);
        q4k_scale_min(hd.y, hd.z, hd.w, 2 * cc + 1, sc1, m1);
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

// ---- Q6K / Q8_0: rows staged in LDS ----

// N dwords of the LDS byte image starting at an even byte offset: the covering aligned
// dwords, shifted by v_alignbyte (a shift of 0 returns the low dword). Reads one dword past
// the last byte, so the staging buffer carries 16 bytes of slack.
template <int N>
__device__ __forceinline__ void lds_dwords(const uint32_t *lds, int off, uint32_t (&o)[N]) {
  const int a = off >> 2, sh = off & 3;
  uint32_t d[N + 1];
#pragma unroll
  for (int i = 0; i <= N; ++i) d[i] = lds[a + i];
#pragma unroll
  for (int i = 0; i < N; ++i) o[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], sh);
}

// LDS position (floats) of input element e: pads that spread the lanes' first reads over
// the banks. Q6K lane (superblock sb, quarter cc) reads 16-float runs at 256 sb + 128 (cc
// >> 1) + 32 g + 16 (cc & 1); Q8_0 lane reads the 32-float block lane (+ 64 k).
template <int kFmt>
__device__ __forceinline__ int xs_pos(int e) {
  if constexpr (kFmt == kWQ6K) return e + 4 * ((e >> 8) + 2 * (e >> 7));
  else return e + 4 * (e >> 5);
}
template <int kFmt>
constexpr int xs_floats(int in) {
  return kFmt == kWQ6K ? in + 4 * (in / 256 + 2 * (in / 128)) : in + 4 * (in / 32);
}

template <int kFmt, int kChunks, int kOprojRowsPerWave>
__global__ __launch_bounds__(256) void oproj_staged_kernel(OprojArgs a) {
  static_assert(kFmt == kWQ6K || kFmt == kWQ8_0, "Q6K or Q8_0");
  constexpr int kIn = 4096 * kChunks;
  constexpr int kRowBytes = kIn / block_elems(kFmt) * block_bytes(kFmt);
  static_assert(kRowBytes % 16 == 0, "rows must be whole 16-byte units");
  constexpr int kRows = kOprojWaves * kOprojRowsPerWave;
  constexpr int kRow16 = kRowBytes / 16;
  __shared__ __attribute__((aligned(16))) float xs[xs_floats<kFmt>(kIn)];
  __shared__ __attribute__((aligned(16))) uint32_t wsm[kRows * kRowBytes / 4 + 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rg0 = blockIdx.x * kRows;  // the workgroup's first row
  const int b = blockIdx.y;
  // the gated input and the rows' bytes: every load goes out before any is used
  constexpr int kIn4 = kIn / 1024;
  float4 x0[kIn4], g0[kIn4];
#pragma unroll
  for (int k = 0; k < kIn4; ++k) {
    x0[k] = reinterpret_cast<const float4 *>(a.attn + (int64_t)b * kIn)[tid + 256 * k];
    g0[k] = a.gate != nullptr
                ? reinterpret_cast<const float4 *>(a.gate + (int64_t)b * kIn)[tid + 256 * k]
                : float4{0.f, 0.f, 0.f, 0.f};
  }
  // the rows' bytes: up to 8 units of 16 B per thread in flight (more would spill), so
  // the widest shapes copy in two rounds
  constexpr int kTotal = kRows * kRow16;
  constexpr int kPer = (kTotal + 255) / 256;
  constexpr int kRound = kPer > 8 ? (kPer + 1) / 2 : kPer;
  auto load_round = [&](int k0, uint4 (&wv)[kRound]) {
#pragma unroll
    for (int k = 0; k < kRound; ++k) {
      // every thread loads (a clamped unit past the end), so that no load sits in a branch
      const int u = min(tid + 256 * (k0 + k), kTotal - 1);
      const int r = u / kRow16, row = rg0 + r < a.out_dim ? rg0 + r : a.out_dim - 1;
      wv[k] = reinterpret_cast<const uint4 *>(a.w + (int64_t)row * kRowBytes)[u - r * kRow16];
    }
  };
  auto store_round = [&](int k0, const uint4 (&wv)[kRound]) {
#pragma unroll
    for (int k = 0; k < kRound; ++k) {
      const int u = tid + 256 * (k0 + k);
      if (k0 + k < kPer && u < kTotal) reinterpret_cast<uint4 *>(wsm)[u] = wv[k];
    }
  };
  {
    uint4 wv[kRound];
    load_round(0, wv);
#pragma unroll
    for (int k = 0; k < kIn4; ++k) {
      float4 x = x0[k];
      if (a.gate != nullptr) {
        x.x *= fast_sigmoid(g0[k].x);
        x.y *= fast_sigmoid(g0[k].y);
        x.z *= fast_sigmoid(g0[k].z);
        x.w *= fast_sigmoid(g0[k].w);
      }
      *reinterpret_cast<float4 *>(xs + xs_pos<kFmt>(4 * (tid + 256 * k))) = x;
    }
    store_round(0, wv);
  }
  if constexpr (kRound < kPer) {
    uint4 wv[kRound];
    load_round(kRound, wv);
    store_round(kRound, wv);
  }
  if (tid < 4) wsm[kRows * kRowBytes / 4 + tid] = 0u;  // the slack lds_dwords may read
  __syncthreads();

  float acc[kOprojRowsPerWave];
#pragma unroll
  for (int r = 0; r < kOprojRowsPerWave; ++r) acc[r] = 0.0f;
  if constexpr (kFmt == kWQ6K) {
    const int cc = lane & 3, hf = cc >> 1, c1 = cc & 1;
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch) {
      const int sb = 16 * ch + (lane >> 2);
      // the 4 runs of 16 inputs this lane weighs: elements 256 sb + 128 hf + 32 g + 16 c1
      float xv[4][16], sx[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float *xr = xs + xs_pos<kFmt>(256 * sb + 128 * hf + 32 * g + 16 * c1);
        sx[g] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 v4 = reinterpret_cast<const float4 *>(xr)[i];
          xv[g][4 * i] = v4.x; xv[g][4 * i + 1] = v4.y; xv[g][4 * i + 2] = v4.z; xv[g][4 * i + 3] = v4.w;
          sx[g] += (v4.x + v4.y) + (v4.z + v4.w);
        }
      }
#pragma unroll
      for (int r = 0; r < kOprojRowsPerWave; ++r) {
        const int B = (wave * kOprojRowsPerWave + r) * kRowBytes + 210 * sb;
        uint32_t qa[4], qb[4], qh[4], scw[2], dw[1];
        lds_dwords(wsm, B + 64 * hf + 16 * c1, qa);       // low nibbles of groups 0, 2
        lds_dwords(wsm, B + 64 * hf + 32 + 16 * c1, qb);  // low nibbles of groups 1, 3
        lds_dwords(wsm, B + 128 + 32 * hf + 16 * c1, qh); // bit pairs of groups 0..3
        lds_dwords(wsm, B + 192 + 8 * hf, scw);           // scales 8 hf .. 8 hf + 7
        lds_dwords(wsm, B + 208, dw);                     // d
        const float d = f16_to_f32((uint16_t)(dw[0] & 0xFFFFu));
        float part = 0.0f;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          // scale 8 hf + 2 g + c1, of elements 128 hf + 32 g + 16 c1 ..: byte 2 g + c1 of
          // the pair, in dword g / 2
          const float sc = (float)(int8_t)(uint8_t)(scw[g >> 1] >> (8 * (((2 * g) & 3) + c1)));
          float p2[2] = {0.0f, 0.0f};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const uint32_t src = (g & 1) ? qb[k] : qa[k];
            const uint32_t code = ((src >> (4 * (g >> 1))) & 0x0F0F0F0Fu) |
                                  (((qh[k] >> (2 * g)) & 0x03030303u) << 4);
            float cf[4];
            bytes_to_f32(code, cf);
#pragma unroll
            for (int i = 0; i < 4; ++i) p2[k & 1] = fmaf(cf[i], xv[g][4 * k + i], p2[k & 1]);
          }
          // codes are stored + 32
          part = fmaf(d * sc, (p2[0] + p2[1]) - 32.0f * sx[g], part);
        }
        acc[r] += part;
      }
    }
  } else {
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch) {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int blk = 128 * ch + lane + 64 * k;
        const float *xr = xs + xs_pos<kFmt>(32 * blk);
        float xv[32], sx = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float4 v4 = reinterpret_cast<const float4 *>(xr)[i];
          xv[4 * i] = v4.x; xv[4 * i + 1] = v4.y; xv[4 * i + 2] = v4.z; xv[4 * i + 3] = v4.w;
          sx += (v4.x + v4.y) + (v4.z + v4.w);
        }
#pragma unroll
        for (int r = 0; r < kOprojRowsPerWave; ++r) {
          const int B = (wave * kOprojRowsPerWave + r) * kRowBytes + 34 * blk;
          uint32_t dw[1], qw[8];
          lds_dwords(wsm, B, dw);
          lds_dwords(wsm, B + 2, qw);
          const float d = f16_to_f32((uint16_t)(dw[0] & 0xFFFFu));
          float p2[2] = {0.0f, 0.0f};
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            float cf[4];
            bytes_to_f32(qw[q] ^ 0x80808080u, cf);  // int8 code + 128
#pragma unroll
            for (int i = 0; i < 4; ++i) p2[q & 1] = fmaf(cf[i], xv[4 * q + i], p2[q & 1]);
          }
          acc[r] = fmaf(d, (p2[0] + p2[1]) - 128.0f * sx, acc[r]);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kOprojRowsPerWave; ++r) {
    const float y = wave64_sum(acc[r]);
    const int row = rg0 + wave * kOprojRowsPerWave + r;
    if (lane == 0 && row < a.out_dim) a.out[(int64_t)b * a.out_dim + row] = y;
  }
}

}  // namespace

int launch_oproj(const float *attn, const float *gate, const uint8_t *w, int w_type, float *out,
                 int batch, int in_dim, int out_dim, hipStream_t s) {
  if (w_type != kWQ4K && w_type != kWQ5K && w_type != kWQ6K && w_type != kWQ8_0)
    return set_error(PKV_ERR_UNSUPPORTED, "gated o_proj: weight type must be Q8_0 (8), Q4K (12), "
                                          "Q5K (13) or Q6K (14)");
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
  const int shape = (in_dim / 4096) * 4 + rows_per_wave;  // 5, 6, 9, 10
#define PKV_OPROJ_CASES(KERNEL, FMT)                                                    \
  switch (shape) {                                                                    \
    case 5: hipLaunchKernelGGL((KERNEL<FMT, 1, 1>), grid, dim3(256), 0, s, a); break; \
    case 6: hipLaunchKernelGGL((KERNEL<FMT, 1, 2>), grid, dim3(256), 0, s, a); break; \
    case 9: hipLaunchKernelGGL((KERNEL<FMT, 2, 1>), grid, dim3(256), 0, s, a); break; \
    default: hipLaunchKernelGGL((KERNEL<FMT, 2, 2>), grid, dim3(256), 0, s, a); break; \
  }
  switch (w_type) {
    case kWQ4K: PKV_OPROJ_CASES(oproj_k45_kernel, kWQ4K); break;
    case kWQ5K: PKV_OPROJ_CASES(oproj_k45_kernel, kWQ5K); break;
    case kWQ6K: PKV_OPROJ_CASES(oproj_staged_kernel, kWQ6K); break;
    default: PKV_OPROJ_CASES(oproj_staged_kernel, kWQ8_0); break;
  }
#undef PKV_OPROJ_CASES
  PKV_HIP(hipGetLastError());
  return PKV_OK;
}

}  // namespace pkv
