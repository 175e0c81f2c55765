// Split-K decode plumbing shared by the decode kernels (Q4K MFMA, Q8_0): the segment
// table of one launch, and the kernel that merges the partials of each output row and
// adds the appended key of a fused decode step. Include-only; every symbol has
// internal linkage.
//
// Partial layout, one slot per piece of work (a workgroup's blocks of one segment):
// part[slot][16 heads][256]: the un-normalised output in tile order (entry 16 T + n
// holds element tile_e(T, n)); ml[slot][16 heads]: the running max m (log2 units) and the
// sum l of 2^(score - m). A row is 1 KB, so the combine's 32-entry slices each fill one
// 128-byte line, and a head's (m, l) pairs of all partials are contiguous.
#pragma once
#include <type_traits>

#include "pkv_internal.hpp"

namespace pkv {
namespace {

constexpr float kSplitClampL2 = 100.0f * 1.4426950408889634f;  // +-100 nats in log2 units
constexpr int kPartRow = 256;  // floats per partial row

// e (0..255) of tile-order entry 16 T + n
__device__ __forceinline__ int tile_e(int T, int n) {
  const int h = T >> 3, byte = (T >> 1) & 3, hl = T & 1;
  const int c = 2 * h + (n >> 3);
  return 64 * c + 32 * hl + 4 * (n & 7) + byte;
}
// tile-order entry of element e (the inverse of tile_e)
__host__ __device__ __forceinline__ int tile_index(int e) {
  const int c = e >> 6, hl = (e >> 5) & 1, r = e & 31;
  const int n = 8 * (c & 1) + (r >> 2), T = 8 * (c >> 1) + 2 * (r & 3) + hl;
  return 16 * T + n;
}

// One launch serves up to kMaxSegs segments: the batch rows of one cache, or the
// sequences of a batched decode step (each with its own cache and length), or the pages
// of paged sequences. Every piece of work (a workgroup's blocks of one segment) writes
// one split-K partial; the combine merges the partials of each output row.
constexpr int kMaxSegs = 32;
struct DecodeSeg {
  uint8_t *k, *v;  // K and V rows of token 0, KV head 0 (rows of head 1 follow at rs_h)
  int64_t seq_k;   // keys held in the cache before this step's append (all attended)
  int64_t t_new;   // row the fused step writes
  int nblk;
  int wg0;         // first workgroup with blocks of this segment
  int qi;          // query / output row of the segment (several segments may share one:
                   // the pages of a paged sequence, merged by the combine)
  int voff;        // stream mode: first block of the segment on the virtual block line
};
struct DecodeSegIn {
  uint8_t *k, *v;
  int64_t seq_k;  // keys after the append (fused) or in the cache
};
// Sum over the 64 lanes of a wave, every lane getting it: DPP moves within rows of 16,
// then v_permlane16_swap and v_permlane32_swap across them (no LDS round trips).
__device__ __forceinline__ float wave_sum(float x) {
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

// Sum (max) over the lanes l, l ^ 8, l ^ 16, l ^ 32 of a wave, every one of them getting it
// (DPP row rotate by 8, then the row-pair and half swaps): the reduction over the 8 partial
// slices a wave holds, with the lane's float4 of entries (l % 8) fixed. The tree order is
// fixed, so the result does not depend on timing.
__device__ __forceinline__ float slices_sum(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, x),
                                                            __builtin_bit_cast(int, x), 0x128, 0xF,
                                                            0xF, false));  // row_ror:8
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
__device__ __forceinline__ float slices_max(float x) {
  x = fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, x),
                                                                    __builtin_bit_cast(int, x), 0x128,
                                                                    0xF, 0xF, false)));
  {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    x = fmaxf(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1));
  }
  {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    x = fmaxf(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1));
  }
  return x;
}

// The end of a (head, 32-entry slice) merge, shared by both combine forms so that they
// give the same bits. 256 threads: thread (ps, g4) = (tid / 8, tid % 8) holds its slice
// of partials' running max m_loc (log2 units), sums acc (entries 4 g4 .. 4 g4 + 3 of the
// slice) and lacc, and qk, its term of the new key's q . k (0 without one). The new key's
// score and weight join the max; threads 0-31 then hold entry tid of the slice: returns
// sum / L for it (vnew: that entry of the new key's V row). Every thread of the workgroup
// (256 or more) calls it: two barriers.
struct FinishSmem {
  float dotp[4], mw[4], lw[4];
  float4 accw[4][8];
};
__device__ __forceinline__ float combine_finish(FinishSmem &t, int tid, bool merger, float m_loc,
                                                float4 acc, float lacc, float qk, bool has_new,
                                                float sl2, float vnew) {
  const int w = tid >> 6, g4 = tid & 7;
  const float d = wave_sum(qk);
  const float mw = slices_max(m_loc);
  if (merger && (tid & 63) == 0) {
    t.dotp[w] = d;
    t.mw[w] = mw;
  }
  __syncthreads();
  const float s_new = has_new ? fminf(fmaxf((t.dotp[0] + t.dotp[1] + t.dotp[2] + t.dotp[3]) * sl2,
                                            -kSplitClampL2), kSplitClampL2)
                              : -INFINITY;
  const float M = fmaxf(fmaxf(fmaxf(s_new, t.mw[0]), fmaxf(t.mw[1], t.mw[2])), t.mw[3]);
  const float f = (m_loc == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_loc - M);
  const float ax = slices_sum(acc.x * f), ay = slices_sum(acc.y * f), az = slices_sum(acc.z * f),
              aw = slices_sum(acc.w * f), al = slices_sum(lacc * f);
  if (merger && (tid & 63) < 8) {
    t.accw[w][g4] = float4{ax, ay, az, aw};
    if (g4 == 0) t.lw[w] = al;
  }
  __syncthreads();
  float r = 0.0f;
  if (tid < 32) {
    const float *a0 = reinterpret_cast<const float *>(&t.accw[0][0]);
    float sum = ((a0[tid] + a0[32 + tid]) + (a0[64 + tid] + a0[96 + tid]));
    float L = ((t.lw[0] + t.lw[1]) + (t.lw[2] + t.lw[3]));
    const float f_new = (s_new == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(s_new - M);
    L += f_new;
    if (has_new) sum += f_new * vnew;
    r = L > 0.0f ? sum / L : 0.0f;
  }
  return r;
}

// out[b][h][e] = (sum_w o_w 2^(m_w - M) + [new key]) / (sum_w l_w 2^(m_w - M) + [new key]).
// One workgroup per (head, 32-entry slice of the tile-order row, batch): thread (ps, g4)
// reads a float4 of entries and the (m, l) pair of every partial in slice ps of the
// partials. Every load of the first round goes out before the new key's q and dq and
// before any is used, so the kernel waits for memory once. Slices keep their own running
// max and merge through LDS. For a fused decode step the appended key enters here, from
// its exactly dequantized K and V rows: score = clamp(q . k_new * scale), weight
// 2^(score - M).
constexpr int kCombSlices = 32;  // partial slices (8 threads each)
constexpr int kCombChunk = 8;    // partials per slice per round
// The output-row table is sized at compile time: one row for a single cache of batch 1
// (the common launch carries the small argument block), kMaxSegs otherwise.
template <int kRows>
struct CombineArgsT {
  const float *part;      // [wg][16][kPartRow]
  const float2 *ml;       // [wg][16] (m, l)
  const float *q, *dq;    // [nseg][16][256], [nseg][4][256] or null
  float *out;             // [nseg][16][256]
  float sl2;
  int wg0[kRows];  // output row b merges partials [wg0[b], wg1[b])
  int wg1[kRows];
};
using CombineArgs = CombineArgsT<kMaxSegs>;
template <int kRows>
__global__ __launch_bounds__(256) void decode_combine_kernel(CombineArgsT<kRows> c) {
  __shared__ FinishSmem fs;
  const int h = blockIdx.x >> 3, i0 = 32 * (blockIdx.x & 7), b = blockIdx.y;
  const int tid = threadIdx.x, ps = tid >> 3, g4 = tid & 7;
  const float *dq = c.dq;
  const float sl2 = c.sl2;
  const int wbeg = c.wg0[b], nwg = c.wg1[b] - wbeg;
  const float *P = c.part + ((int64_t)wbeg * 16 + h) * kPartRow + i0 + 4 * g4;
  const float2 *ML = c.ml + (int64_t)wbeg * 16 + h;
  const int per = (nwg + kCombSlices - 1) / kCombSlices;
  const int w0 = ps * per, w1 = w0 + per < nwg ? w0 + per : nwg;
  float2 mlv[kCombChunk];
  float4 ov[kCombChunk];
  auto load_round = [&](int w) {
#pragma unroll
    for (int x = 0; x < kCombChunk; ++x) {
      const bool ok = w + x < w1;
      mlv[x] = ok ? ML[(int64_t)(w + x) * 16] : float2{-INFINITY, 0.0f};
      ov[x] = ok ? *reinterpret_cast<const float4 *>(P + (int64_t)(w + x) * 16 * kPartRow)
                 : float4{0.f, 0.f, 0.f, 0.f};
    }
  };
  load_round(w0);
  // the new key's q . k_new products, loaded after the partials (reduced further down)
  float qv = 0.0f, kv = 0.0f;
  if (dq != nullptr) {
    qv = c.q[((int64_t)b * 16 + h) * 256 + tid];
    kv = dq[((int64_t)b * 4 + (h >> 3)) * 256 + tid];
  }
  float m_loc = -INFINITY, lacc = 0.0f;
  float4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int w = w0; w < w1; w += kCombChunk) {
    if (w != w0) load_round(w);
    float mc = m_loc;
#pragma unroll
    for (int x = 0; x < kCombChunk; ++x) mc = fmaxf(mc, mlv[x].x);
    if (mc != -INFINITY) {
      const float r = (m_loc == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_loc - mc);
      acc.x *= r;
      acc.y *= r;
      acc.z *= r;
      acc.w *= r;
      lacc *= r;
#pragma unroll
      for (int x = 0; x < kCombChunk; ++x) {
        const float f = (mlv[x].x == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mlv[x].x - mc);
        acc.x += f * ov[x].x;
        acc.y += f * ov[x].y;
        acc.z += f * ov[x].z;
        acc.w += f * ov[x].w;
        lacc += f * mlv[x].y;
      }
      m_loc = mc;
    }
  }
  const int e = tile_e((i0 + (tid & 31)) >> 4, (i0 + (tid & 31)) & 15);
  const float vnew = (dq != nullptr && tid < 32) ? dq[((int64_t)b * 4 + 2 + (h >> 3)) * 256 + e] : 0.0f;
  const float r = combine_finish(fs, tid, true, m_loc, acc, lacc, qv * kv, dq != nullptr, sl2, vnew);
  if (tid < 32) c.out[((int64_t)b * 16 + h) * 256 + e] = r;
}

// Launch the combine over n output rows (grid: 128 (head, slice) workgroups per row).
static inline int launch_combine(const CombineArgs &c, int n, hipStream_t s) {
  if (n == 1) {
    CombineArgsT<1> c1;
    c1.part = c.part;
    c1.ml = c.ml;
    c1.q = c.q;
    c1.dq = c.dq;
    c1.out = c.out;
    c1.sl2 = c.sl2;
    c1.wg0[0] = c.wg0[0];
    c1.wg1[0] = c.wg1[0];
    hipLaunchKernelGGL(decode_combine_kernel<1>, dim3(16 * 8, 1u), dim3(256), 0, s, c1);
  } else {
    hipLaunchKernelGGL(decode_combine_kernel<kMaxSegs>, dim3(16 * 8, (unsigned)n), dim3(256), 0,
                       s, c);
  }
  PKV_HIP(hipGetLastError());
  return PKV_OK;
}

}  // namespace

// Rows are addressed with 32-bit offsets (key * row stride) from a per-head base.
static inline bool decode_rows_fit(int64_t seq_k, int64_t rs_t) {
  return rs_t < (1 << 24) && seq_k < (1 << 24) && (uint64_t)seq_k * (uint64_t)rs_t < (1ull << 32);
}

}  // namespace pkv
