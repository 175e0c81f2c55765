// Latency-oriented, bit-exact Q4K quantizer (candle BlockQ4K::from_float with
// make_qkx1_quants(15, 5), restated; reference call site
// paramecia-model/src/qwen3_next.rs:486-487): 256 threads per 256-element superblock,
// one element per lane, 32 lanes per sub-block. The two f32 sums of make_qkx1_quants
// accumulate in element order in the reference, so each sub-block's 32-term chain is
// replayed in order, moving across its lanes; the element-wise work (rounding,
// clamping, products, the final division) runs in parallel. The bytes
// equal those of the 8-lane throughput kernel and of the CPU oracle.
// Include-only; every function keeps a*b+c as two roundings (contraction off).
#pragma once
#include "pkv_scalar.hpp"

namespace pkv {

// (nearest_int(v)).clamp(0, 15), nearest_int being candle's v.round() as i32 (half away
// from zero, NaN -> 0), in two instructions. v_med3_f32 clamps to [0, 15] first; with a
// NaN operand it returns the least of the other two, 0. v_cvt_rpi_i32_f32 then gives
// floor(c + 0.5) without rounding the sum, which on [0, 15] is round half away from zero.
__device__ __forceinline__ int32_t q4_level_i(float v) {
  const float c = __builtin_amdgcn_fmed3f(v, 0.0f, 15.0f);
  int32_t r;
  asm("v_cvt_rpi_i32_f32 %0, %1" : "=v"(r) : "v"(c));
  return r;
}

struct Q4kScratch {
  float red[2][8];
  uint32_t codes[8];
  uint8_t nib[256];
};

// The 32-term sum of each half-wave's terms (lane i of the half holds term i) in element
// order, init first, in registers: the running sum moves up one lane per step (DPP
// wave_shr:1), so after step k lane i holds ((init + t[i-k]) + ...) + t[i]. Lanes 31 and
// 63 end with their half's sum (lane 32 starts its chain from init at step 0, like lane
// 0), which is then read out and given to every lane of the half. No LDS round trip: the
// other waves' block traffic makes those long.
__device__ __forceinline__ float q4k_chain_sum_32(float term, float init) {
#pragma clang fp contract(off)
  float acc = init + term;
#pragma unroll
  for (int k = 1; k < 32; ++k) {
    const int prev = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc), 0x138, 0xF, 0xF, false);
    acc = __builtin_bit_cast(float, prev) + term;
  }
  const int lo = __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 31);
  const int hi = __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 63);
  return __builtin_bit_cast(float, (__lane_id() < 32) ? lo : hi);
}

// All-reduce over the 32 lanes of each half-wave with DPP moves (within 16-lane rows)
// and v_permlane16_swap (between the two rows of a half): a few VALU cycles per step
// instead of an LDS round trip per __shfl_xor. Integer ops, so the order is immaterial.
template <typename Op>
__device__ __forceinline__ int32_t halfwave_allreduce(int32_t x, Op op) {
  x = op(x, __builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
  x = op(x, __builtin_amdgcn_update_dpp(x, x, 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
  x = op(x, __builtin_amdgcn_update_dpp(x, x, 0x141, 0xF, 0xF, false));  // row_half_mirror
  x = op(x, __builtin_amdgcn_update_dpp(x, x, 0x140, 0xF, 0xF, false));  // row_mirror
  const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)x, (uint32_t)x, false, false);
  const uint32_t r0 = r[0], r1 = r[1];  // scalar copies (see the decode kernel's note)
  return op((int32_t)r0, (int32_t)r1);
}

// Barrier over the 256 threads of a quantization: by default the workgroup barrier.
struct Q4kWorkgroupBarrier {
  __device__ __forceinline__ void operator()() const { __syncthreads(); }
};

// x: this thread's element (tid = 32 * sub-block + element); blk: 144 output bytes.
// Called by 256 threads (four waves) together; `bar` synchronises exactly those four
// waves (three times per call).
template <typename Barrier = Q4kWorkgroupBarrier>
static __device__ __forceinline__ void q4k_quantize_superblock_lanes(float x, uint8_t *blk,
                                                                   Q4kScratch *S, int tid,
                                                                   float *deq = nullptr,
                                                                   Barrier bar = Barrier()) {
#pragma clang fp contract(off)
  const int j = tid >> 5, i = tid & 31;
  const auto imin = [](int32_t p, int32_t q) { return p < q ? p : q; };
  const auto imax = [](int32_t p, int32_t q) { return p > q ? p : q; };
  const auto iadd = [](int32_t p, int32_t q) { return p + q; };
  const int32_t kmin = halfwave_allreduce(total_key(x), imin);
  const int32_t kmax = halfwave_allreduce(total_key(x), imax);
  auto from_key = [](int32_t k) {
    return u2f((uint32_t)(k ^ (int32_t)(((uint32_t)(k >> 31)) >> 1)));
  };
  const float mn = from_key(kmin), mx = from_key(kmax);
  float scale = 0.0f, neg_min = 0.0f;
  uint32_t L = 0;
  if (!(mx == mn)) {
    float fmin = fmin_rs(mn, 0.0f);
    float iscale = 15.0f / (mx - fmin);
    scale = 1.0f / iscale;
    for (int t = 0; t < 5; ++t) {
      const int32_t li = q4_level_i(iscale * (x - fmin));
      const bool changed = (uint32_t)li != L;
      L = (uint32_t)li;
      const float sumlx = q4k_chain_sum_32((x - fmin) * (float)li, 0.0f);
      const int32_t l2 = halfwave_allreduce(li * li, iadd);
      scale = sumlx / (float)l2;
      const float sum = q4k_chain_sum_32(x - scale * (float)L, -0.0f);
      fmin = sum / 32.0f;
      if (fmin > 0.0f) fmin = 0.0f;
      iscale = 1.0f / scale;
      // did_change of this sub-block: its half of the wave's ballot
      const uint64_t bal = __ballot(changed);
      const uint32_t mask = (uint32_t)(bal >> (32 * ((tid >> 5) & 1)));
      if (mask == 0u) break;
    }
    neg_min = -fmin;
  }
  if (i == 0) {
    S->red[0][j] = scale;
    S->red[1][j] = neg_min;
  }
  bar();
  // The 16 values come into registers first (four LDS reads, one wait): read inside the
  // fold, each read followed the previous step's uniform branch on a NaN, one LDS round
  // trip per value.
  float rv[2][8];
  {
    const float4 *r4 = reinterpret_cast<const float4 *>(&S->red[0][0]);
    const float4 t0 = r4[0], t1 = r4[1], t2 = r4[2], t3 = r4[3];
    rv[0][0] = t0.x; rv[0][1] = t0.y; rv[0][2] = t0.z; rv[0][3] = t0.w;
    rv[0][4] = t1.x; rv[0][5] = t1.y; rv[0][6] = t1.z; rv[0][7] = t1.w;
    rv[1][0] = t2.x; rv[1][1] = t2.y; rv[1][2] = t2.z; rv[1][3] = t2.w;
    rv[1][4] = t3.x; rv[1][5] = t3.y; rv[1][6] = t3.z; rv[1][7] = t3.w;
    asm volatile("" : "+v"(rv[0][0]), "+v"(rv[0][1]), "+v"(rv[0][2]), "+v"(rv[0][3]),
                 "+v"(rv[0][4]), "+v"(rv[0][5]), "+v"(rv[0][6]), "+v"(rv[0][7]),
                 "+v"(rv[1][0]), "+v"(rv[1][1]), "+v"(rv[1][2]), "+v"(rv[1][3]),
                 "+v"(rv[1][4]), "+v"(rv[1][5]), "+v"(rv[1][6]), "+v"(rv[1][7]));
  }
  float max_scale = 0.0f, max_min = 0.0f;  // fold from +0, NaN-dropping maxNum
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) {
    max_scale = fmax_rs(rv[0][jj], max_scale);
    max_min = fmax_rs(rv[1][jj], max_min);
  }
  const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
  const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
  const int32_t ls32 = nearest_int(inv_scale * scale), lm32 = nearest_int(inv_min * neg_min);
  const uint32_t ls = (uint8_t)(ls32 < 63 ? ls32 : 63), lm = (uint8_t)(lm32 < 63 ? lm32 : 63);
  const uint16_t dh = f32_to_f16(max_scale / 63.0f), mh = f32_to_f16(max_min / 63.0f);
  uint32_t q = 0;
  const float dd = f16_to_f32(dh) * (float)ls;
  if (dd != 0.0f) {
    const float dm = f16_to_f32(mh) * (float)lm;
    q = (uint32_t)q4_level_i((x + dm) / dd);
  }
  if (deq != nullptr) {  // to_float of this element: d * sc * q - dmin * m (two roundings)
    const float d1 = f16_to_f32(dh) * (float)ls, m1 = f16_to_f32(mh) * (float)lm;
    *deq = d1 * (float)q - m1;
  }
  if (i == 0) S->codes[j] = ls | (lm << 8);
  S->nib[tid] = (uint8_t)q;
  bar();
  if (tid < 32) {  // qs[32c + l] = L_{2c}[l] | L_{2c+1}[l] << 4, 4 bytes per thread
    uint32_t w = 0;
#pragma unroll
    for (int bb = 0; bb < 4; ++bb) {
      const int byte = 4 * tid + bb, c = byte >> 5, l = byte & 31;
      w |= ((uint32_t)S->nib[64 * c + l] | ((uint32_t)S->nib[64 * c + 32 + l] << 4)) << (8 * bb);
    }
    reinterpret_cast<uint32_t *>(blk + 16)[tid] = w;
  } else if (tid == 32) {
    uint8_t sc[12];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const uint32_t ls_lo = S->codes[jj] & 0xFF, lm_lo = S->codes[jj] >> 8;
      const uint32_t ls_hi = S->codes[jj + 4] & 0xFF, lm_hi = S->codes[jj + 4] >> 8;
      sc[jj] = (uint8_t)(ls_lo | ((ls_hi >> 4) << 6));
      sc[jj + 4] = (uint8_t)(lm_lo | ((lm_hi >> 4) << 6));
      sc[jj + 8] = (uint8_t)((ls_hi & 0xF) | ((lm_hi & 0xF) << 4));
    }
    uint4 hd;
    hd.x = (uint32_t)dh | ((uint32_t)mh << 16);
    hd.y = (uint32_t)sc[0] | ((uint32_t)sc[1] << 8) | ((uint32_t)sc[2] << 16) | ((uint32_t)sc[3] << 24);
    hd.z = (uint32_t)sc[4] | ((uint32_t)sc[5] << 8) | ((uint32_t)sc[6] << 16) | ((uint32_t)sc[7] << 24);
    hd.w = (uint32_t)sc[8] | ((uint32_t)sc[9] << 8) | ((uint32_t)sc[10] << 16) | ((uint32_t)sc[11] << 24);
    *reinterpret_cast<uint4 *>(blk) = hd;
  }
  bar();  // scratch is reused by the next call
}

}  // namespace pkv
