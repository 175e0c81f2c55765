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
#include <cstdlib>
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
// The merge of output row b from partials [wbeg, wbeg + nwg).
__device__ __forceinline__ void combine_row(FinishSmem &fs, const float *part, const float2 *ml,
                                            const float *q, const float *dq, float *out, float sl2,
                                            int wbeg, int nwg, int b) {
  const int h = blockIdx.x >> 3, i0 = 32 * (blockIdx.x & 7);
  const int tid = threadIdx.x, ps = tid >> 3, g4 = tid & 7;
  const float *P = part + ((int64_t)wbeg * 16 + h) * kPartRow + i0 + 4 * g4;
  const float2 *ML = ml + (int64_t)wbeg * 16 + h;
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
  // the new key's q . k_new products and this thread's V value of it, loaded after the
  // partials (reduced further down)
  const int e = tile_e((i0 + (tid & 31)) >> 4, (i0 + (tid & 31)) & 15);
  float qv = 0.0f, kv = 0.0f, vnew = 0.0f;
  if (dq != nullptr) {
    qv = q[((int64_t)b * 16 + h) * 256 + tid];
    kv = dq[((int64_t)b * 4 + (h >> 3)) * 256 + tid];
    if (tid < 32) vnew = dq[((int64_t)b * 4 + 2 + (h >> 3)) * 256 + e];
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
  const float r = combine_finish(fs, tid, true, m_loc, acc, lacc, qv * kv, dq != nullptr, sl2, vnew);
  if (tid < 32) out[((int64_t)b * 16 + h) * 256 + e] = r;
}
template <int kRows>
__global__ __launch_bounds__(256) void decode_combine_kernel(CombineArgsT<kRows> c) {
  __shared__ FinishSmem fs;
  const int b = blockIdx.y;
  combine_row(fs, c.part, c.ml, c.q, c.dq, c.out, c.sl2, c.wg0[b], c.wg1[b] - c.wg0[b], b);
}
// One output row, every argument a scalar: the leading kernel arguments are preloaded into
// SGPRs where the build asks for it, so the first loads wait for no kernel-argument fetch.
__global__ __launch_bounds__(256) void decode_combine1_kernel(const float *part, const float2 *ml,
                                                              const float *q, const float *dq,
                                                              float *out, float sl2, int wbeg,
                                                              int nwg) {
  __shared__ FinishSmem fs;
  combine_row(fs, part, ml, q, dq, out, sl2, wbeg, nwg, 0);
}

// ---- In-launch combine of a one-row decode (the combiner workgroups of a decode launch
// over Workspace::kFusedSlots workgroups).
// Combiner c (grid index nwg + c) merges head c / 8, tile-order entries 32 (c % 8) ..
// +31, as decode_combine_kernel does, inside the decode launch: a combiner is dispatched
// once a decode workgroup has left its CU (the decode workgroups come first in the grid
// and never wait, so they all finish whatever the dispatch order).
// Readiness without flags or cache maintenance: every word a decode workgroup writes for
// the combiners carries the launch's parity in its lowest bit (partial values and (m, l)
// lose that bit; both combine forms clear it, so they give the same bits), written with
// agent-scope (sc1) stores, and each combiner thread polls the very words it merges with
// agent-scope loads until their parity is the launch's. A slot holds either the previous
// launch's words (the other parity) or this launch's: every launch writes every slot it
// uses, and launches on a workspace are ordered on one stream. The launch parity: decode
// workgroups read word kWordGen at their start and use its complement; combiner c keeps
// its own copy in word kWordComb + c and flips it once its merge is done, and combiner 0
// also flips kWordGen then, after every decode workgroup has read it (each one read it
// before writing a partial that combiner 0 has merged). The new rows and the prepared q
// are written early and flagged by words set to the parity after s_waitcnt vmcnt(0). The
// waits are bounded (2^16 polls); a combiner that gives up sets kStatusBarrierTimeout
// (pkv_device_status()), and the words must then be zeroed again (a new workspace).
constexpr int kTailWGs = 128;  // 16 heads x 8 slices of 32 entries
constexpr int kTailThreads = 512;  // threads 0-255 merge, 256-511 only wait
static_assert(kCombSlices * kCombChunk == Workspace::kFusedSlots && kCombSlices * 8 <= kTailThreads,
              "combiner layout: one round of partial loads over the fused slots");
constexpr int kWordGen = 0;      // launch parity seen by the decode workgroups
constexpr int kWordComb = 32;    // + c: combiner c's launch parity
constexpr int kWordRow = 256;    // + r: parity of the launch whose new row r is stored
constexpr int kWordQ = 288;      // + kv: parity of the launch whose prepared q rows are stored
static_assert(kWordComb + kTailWGs <= kWordRow && kWordQ + 2 <= Workspace::kFusedWords, "words");
constexpr int kSC1 = 16;  // buffer cache policy bit: agent-scope coherent access (sc1)

__device__ __forceinline__ void store_sc1(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_sc1(uint32_t *p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_sc1(const float *p) {
  return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t load_sc1(const uint32_t *p) {
  return __hip_atomic_load(const_cast<uint32_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// a partial word with its lowest bit replaced by the launch parity, and back
__device__ __forceinline__ float tag_par(float x, uint32_t par) {
  return __builtin_bit_cast(float, (__builtin_bit_cast(uint32_t, x) & ~1u) | par);
}
__device__ __forceinline__ float untag(float x) {
  return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, x) & ~1u);
}
__device__ __forceinline__ uint32_t par_of(float x) { return __builtin_bit_cast(uint32_t, x) & 1u; }

// The merge is decode_combine_kernel's, step for step (the same slices, partial order and
// sums), so both forms give the same bits.
// The fields a combiner reads: nwg partial slots at part / ml (the fused region), the
// control words, q (or, with kPrep, the prepared q_out), the new rows dq (null without
// a fused append), the output row and the status word.
struct TailArgs {
  int nwg;
  uint32_t *words;
  const float *part;
  const float2 *ml;
  const float *q, *q_out, *dq;
  float *out;
  float sl2;
  unsigned *status;
};
template <bool kPrep>
__device__ __forceinline__ void tail_combine(const TailArgs &a, int c, void *lds) {
  FinishSmem &t = *reinterpret_cast<FinishSmem *>(lds);
  const int nwg = a.nwg;
  const int h = c >> 3, i0 = 32 * (c & 7), kvh = h >> 3;
  const int tid = threadIdx.x, ps = tid >> 3, g4 = tid & 7;
  const bool merger = tid < kCombSlices * 8;  // threads 0-255; waves 4-7 only wait
  const int per = (nwg + kCombSlices - 1) / kCombSlices;  // <= kCombChunk
  const int w0 = ps * per, w1 = w0 + per < nwg ? w0 + per : nwg;
  const bool fused = a.dq != nullptr;
  const uint32_t par = (load_sc1(a.words + kWordComb + c) ^ 1u) & 1u;
  float2 mlv[kCombChunk];
  float4 ov[kCombChunk];
  bool ok = true;
  // the new key's q . k products and this thread's V value of it, loaded during the polls
  // as soon as the wave has seen the new rows' (and prepared q's) words
  const int e_out = tile_e((i0 + (tid & 31)) >> 4, (i0 + (tid & 31)) & 15);
  float qv = 0.0f, kv = 0.0f, vnew = 0.0f;
  if (merger) {
    // Poll the words this thread merges (and, on lanes 0-2, the new-row and prepared-q
    // words every lane reads) until each has this launch's parity.
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(a.part), 0, nwg * 16 * kPartRow * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rm =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float2 *>(a.ml), 0, nwg * 16 * 8, 0x00020000);
    const int cnt = w1 > w0 ? w1 - w0 : 0;  // entries of this thread's slice
    const int lane = tid & 63;
    const uint32_t *xw = (lane < 2 && fused) ? a.words + kWordRow + 2 * lane + kvh
                         : (lane == 2 && kPrep) ? a.words + kWordQ + kvh
                                                : nullptr;
    bool xok = xw == nullptr, have_new = !fused;
    // Two poll rounds in flight: round r + 1's loads go out before round r's words are
    // checked, so a word that lands during a round is seen about half a round trip
    // sooner. Every round reloads every entry (a word, once this launch's, stays so).
    float2 mlb[kCombChunk];
    float4 ovb[kCombChunk];
    uint32_t xa = 0u, xb = 0u;  // each round's copy of the lane's new-row / q word
    const uint32_t *xw_any = xw != nullptr ? xw : a.words;  // (a load with no branch)
    auto issue = [&](float2 (&m)[kCombChunk], float4 (&o)[kCombChunk], uint32_t &xv) {
      xv = load_sc1(xw_any);
#pragma unroll
      for (int x = 0; x < kCombChunk; ++x) {
        const int w = x < cnt ? w0 + x : w0;  // (past cnt: a copy of the first, unused)
        m[x] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rm, (w * 16 + h) * 8, 0, kSC1));
        o[x] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                              rp, ((w * 16 + h) * kPartRow + i0 + 4 * g4) * 4, 0, kSC1));
      }
    };
    const uint32_t pm = par ? 0u : 1u;  // a word is this launch's when its low bit ^ pm is 1
    auto check = [&](const float2 (&m)[kCombChunk], const float4 (&o)[kCombChunk],
                     uint32_t xv) -> bool {
      uint32_t miss = 0u;
#pragma unroll
      for (int x = 0; x < kCombChunk; ++x) {
        const uint32_t mok = (par_of(m[x].x) ^ pm) & (par_of(m[x].y) ^ pm);
        const uint32_t ook = (par_of(o[x].x) ^ pm) & (par_of(o[x].y) ^ pm) &
                             (par_of(o[x].z) ^ pm) & (par_of(o[x].w) ^ pm);
        if (x < cnt && !(mok && ook)) miss |= 1u << x;
      }
      if (!xok) xok = (xv & 1u) == par;
      if (!have_new && __all(xok)) {  // the new rows are stored: their values, once
        qv = kPrep ? load_sc1(a.q_out + h * 256 + tid) : a.q[h * 256 + tid];
        kv = load_sc1(a.dq + kvh * 256 + tid);
        if (tid < 32) vnew = load_sc1(a.dq + (2 + kvh) * 256 + e_out);
        have_new = true;
      }
      return __all(miss == 0u && xok) && have_new;
    };
    bool done = false;
    issue(mlv, ov, xa);
    for (int it = 0; it < (1 << 15) && !done; ++it) {
      issue(mlb, ovb, xb);
      if (check(mlv, ov, xa)) {
        done = true;
        break;
      }
      issue(mlv, ov, xa);
      if (check(mlb, ovb, xb)) {
#pragma unroll
        for (int x = 0; x < kCombChunk; ++x) {
          mlv[x] = mlb[x];
          ov[x] = ovb[x];
        }
        done = true;
      }
    }
#pragma unroll
    for (int x = 0; x < kCombChunk; ++x)
      if (x >= cnt) {  // no partial: an empty entry
        mlv[x] = float2{-INFINITY, 0.0f};
        ov[x] = float4{0.f, 0.f, 0.f, 0.f};
      }
    ok = done;
#pragma unroll
    for (int x = 0; x < kCombChunk; ++x) {
      mlv[x] = float2{untag(mlv[x].x), untag(mlv[x].y)};
      ov[x] = float4{untag(ov[x].x), untag(ov[x].y), untag(ov[x].z), untag(ov[x].w)};
    }
  }
  float m_loc = -INFINITY, lacc = 0.0f;
  float4 acc = {0.f, 0.f, 0.f, 0.f};
  if (merger) {
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
  // every merging wave has seen this launch's words: the launch parity flips (combiner 0
  // also flips the decode workgroups' copy, which they have all read by now)
  if (tid == 0) {
    store_sc1(a.words + kWordComb + c, par);
    if (c == 0) store_sc1(a.words + kWordGen, par);
  }
  const float r = combine_finish(t, tid, merger, m_loc, acc, lacc, qv * kv, fused, a.sl2, vnew);
  if (merger && !ok && (tid & 63) == 0)
    __hip_atomic_fetch_or(a.status, kStatusBarrierTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (tid < 32) a.out[h * 256 + e_out] = r;
}

// The in-launch combine of one-row decodes is on unless PKV_DECODE_FUSE=0 (the separate
// combine kernel, kept for comparison).
static inline bool decode_fuse_enabled() {
  static const bool on = [] {
    const char *e = getenv("PKV_DECODE_FUSE");
    return !(e && e[0] == '0');
  }();
  return on;
}

// Launch the combine over n output rows (grid: 128 (head, slice) workgroups per row).
static inline int launch_combine(const CombineArgs &c, int n, hipStream_t s) {
  if (n == 1) {
    hipLaunchKernelGGL(decode_combine1_kernel, dim3(16 * 8, 1u), dim3(256), 0, s, c.part, c.ml,
                       c.q, c.dq, c.out, c.sl2, c.wg0[0], c.wg1[0] - c.wg0[0]);
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
// The decode kernels' packed row strides: rs_t (< 2^24, decode_rows_fit) | rs_h << 24
// (rs_h < 2^40, decode_head_stride_fits).
static inline bool decode_head_stride_fits(int64_t rs_h) { return rs_h >= 0 && rs_h < (1ll << 40); }
static inline uint64_t decode_strides(int64_t rs_t, int64_t rs_h) {
  return (uint64_t)rs_t | ((uint64_t)rs_h << 24);
}

}  // namespace pkv
