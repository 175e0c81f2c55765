// Decode attention over a Q8_0 cache for the Qwen3-Next full-attention shape (16 query
// heads, 2 KV heads, head_dim 256), gfx950.
//
// Role: the reference's only GPU attention over quantized K/V, flash_attn_q8
// (paramecia-model/src/ops.rs:756-792, called at qwen3_next.rs:2531-2561), for a decode
// step (one query that sees every key), and the CPU SDPA it replaces
// (qwen3_next.rs:2580-2605). A Q8_0 row is 8 blocks of {f16 d, 32 x int8}: element e is
// int8 * d of block e / 32 (BlockQ8_0::to_float).
//
// Work split: a workgroup of 512 threads owns a contiguous key range of one segment
// (one cache's batch row, or one sequence of a batched decode step) and both KV heads;
// threads 0-255 take KV head 0, threads 256-511 head 1. The range streams through LDS
// in chunks of 32 keys (K and V rows of both heads, 34.8 KB; 16 keys up to 8192 cached
// keys): QK with one or two threads per (query head, key), an online softmax per query
// head over the chunk, then PV with one
// thread per output element e for the group's 8 query heads. Each workgroup writes one
// split-K partial in tile order; decode_combine_kernel merges them (and the new key of
// a fused step). Dequantization is exact (int8 * d in f32, as the reference's to_float),
// all products and sums f32.
//
// Fused append: workgroups 0 .. 4 * segments - 1 first quantize one new row each
// (BlockQ8_0::from_float, bit-exact) and publish it dequantized for the combine.
#include <cstring>
#include <vector>

#include "pkv_decode_split.hpp"
#include "pkv_q8_common.hpp"
#include "pkv_scalar.hpp"

namespace pkv {
namespace {

constexpr int kQ8Row = 272;    // bytes of one head's row: 8 blocks x 34
constexpr int kQ8Chunk = 32;   // keys per LDS chunk (16 for short caches)
constexpr int kQ8Threads = 512;
constexpr int kQ8RowWords = kQ8Row / 4;  // 68 dwords, 16-byte aligned rows (272 = 17 x 16)

// The scalar fields come first: the kernels read them through the scalar cache, and
// ahead of the segment table they share its first lines with segment 0.
struct Q8Args {
  int nseg, nwg, kpw;  // segments, workgroups, keys per workgroup (a multiple of 32)
  float sl2;
  int64_t rs_t, rs_h;
  const float *q;              // [nseg][16][256]
  const float *k_new, *v_new;  // [nseg][2][256] or null
  float *part;                 // [nwg][16][kPartRow]
  float2 *ml;                  // [nwg][16] running max and sum
  float *dq;                   // [nseg][4][256]
  // Paged mode (dseg non-null): the segment table lives in device memory, segment s
  // owning workgroups [s * wps, (s + 1) * wps); the seg array is unused
  const DecodeSeg *dseg;
  int wps;
  DecodeSeg seg[kMaxSegs];
};

template <int kChunk>
struct alignas(16) Q8Smem {
  uint32_t k[2][kChunk][kQ8RowWords];  // [kv][key][dword]
  uint32_t v[2][kChunk][kQ8RowWords];
  float q[16][256];
  float p[2][kChunk][8];  // weights [kv][key][head of the group]
  float alpha[2][8];      // rescale of the running sums for this chunk
};

// BlockQ8_0::from_float of one 256-element row by 256 threads (thread e owns element
// e): d = amax / 127 of its 32-block, q = round(x / d) saturated to i8, d stored as
// f16. Returns the dequantized element (q * f16(d), the reference's to_float).
__device__ float q8_quantize_row_lanes(float x, uint8_t *row, int e) {
#pragma clang fp contract(off)
  float amax = __builtin_fabsf(x);
#pragma unroll
  for (int o = 16; o >= 1; o >>= 1) amax = fmax_rs(amax, __shfl_xor(amax, o, 32));
  // amax: maxNum fold from +0 of |x| over the block; the order does not matter for
  // maxNum, so the butterfly equals the sequential fold.
  amax = fmax_rs(amax, 0.0f);
  const float d = amax / 127.0f;
  const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
  const int32_t qv = rs_as_i8(__builtin_roundf(x * id));
  const uint16_t dh = f32_to_f16(d);
  uint8_t *blk = row + (e >> 5) * 34;
  blk[2 + (e & 31)] = (uint8_t)qv;
  if ((e & 31) == 0) {
    blk[0] = (uint8_t)(dh & 0xFF);
    blk[1] = (uint8_t)(dh >> 8);
  }
  return (float)qv * f16_to_f32(dh);
}

// exact f16 -> f32 of the low (hi = 0) or high half of a dword (hardware conversion)
__device__ __forceinline__ float h16(uint32_t w, int hi) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(hi ? (w >> 16) : (w & 0xFFFF)));
}

// kChunk keys per LDS chunk. 32: one QK thread per (query head, key) over all 256
// dimensions. 16 (short caches, twice the workgroups): two threads per (query head, key),
// each over four of the eight blocks, their sums added by a lane exchange; every
// workgroup then does half the work of a 32-key one, so a launch with one chunk per
// workgroup ends sooner.
template <int kChunk>
__global__ __launch_bounds__(kQ8Threads) void q8_decode_kernel(Q8Args a) {
  __shared__ Q8Smem<kChunk> sm;
  const int tid = threadIdx.x, half = tid >> 8, t = tid & 255;
  const int wg = blockIdx.x;
  int b = 0;
  DecodeSeg sgv;
  if (a.dseg != nullptr) {
    b = wg / a.wps;
    sgv = a.dseg[b];
  } else {
    while (b + 1 < a.nseg && wg >= a.seg[b + 1].wg0) ++b;
    sgv = a.seg[b];
  }
  const DecodeSeg &sg = sgv;
  const int64_t k0 = (int64_t)(wg - sg.wg0) * a.kpw;
  const int64_t k1 = k0 + a.kpw < sg.seq_k ? k0 + a.kpw : sg.seq_k;

  // ---- fused append: new row r = 4 s + 2 p + kv (K p = 0, V p = 1), one per workgroup
  if (a.k_new != nullptr && half == 0) {
    for (int row = wg; row < 4 * a.nseg; row += a.nwg) {
      const int rs = row >> 2, p = (row >> 1) & 1, kvr = row & 1;
      const float x = (p ? a.v_new : a.k_new)[((int64_t)rs * 2 + kvr) * 256 + t];
      const DecodeSeg &rg = a.seg[rs];
      uint8_t *dst = (p ? rg.v : rg.k) + rg.t_new * a.rs_t + kvr * a.rs_h;
      a.dq[(int64_t)row * 256 + t] = q8_quantize_row_lanes(x, dst, t);
    }
  }

  // ---- chunk staging: K and V rows of both heads, 2 x 2 x kChunk x 68 dwords, loaded
  // into registers, then written to LDS
  constexpr int kWords = 2 * kChunk * kQ8RowWords;  // per tensor
  constexpr int kPer = (kWords + kQ8Threads - 1) / kQ8Threads;
  uint32_t kv_[2][kPer];
  const auto load_chunk = [&](int64_t c0, int nk) {
#pragma unroll
    for (int x = 0; x < kPer; ++x) {
      const int i = tid + x * kQ8Threads;
      const int kvh = i / (kChunk * kQ8RowWords), r = i % (kChunk * kQ8RowWords);
      const int key = r / kQ8RowWords, w = r % kQ8RowWords;
      const bool ok = i < kWords && key < nk;
      const int64_t off = (c0 + (ok ? key : 0)) * a.rs_t + kvh * a.rs_h + 4 * w;
      kv_[0][x] = ok ? *reinterpret_cast<const uint32_t *>(sg.k + off) : 0u;
      kv_[1][x] = ok ? *reinterpret_cast<const uint32_t *>(sg.v + off) : 0u;
    }
  };
  const auto chunk_keys = [&](int64_t c0) { return (int)(k1 - c0 < kChunk ? k1 - c0 : kChunk); };

  // ---- q of the 16 heads into LDS; the first chunk's loads are issued behind q's, so
  // that both are in flight together
  {
    const float4 *q4 = reinterpret_cast<const float4 *>(a.q + (int64_t)sg.qi * 16 * 256);
    const float4 qa = q4[tid], qb = q4[tid + 512];
    if (k0 < k1) load_chunk(k0, chunk_keys(k0));
    float4 *s4 = reinterpret_cast<float4 *>(&sm.q[0][0]);
    s4[tid] = qa;
    s4[tid + 512] = qb;
  }

  // QK role: (head hh of the group, key kk of the chunk[, block half dh]); PV role:
  // element e = t
  constexpr int kSplit = 32 / kChunk;  // threads per (head, key)
  const int hh = t >> 5, kk = (t & 31) / kSplit, dh = t & (kSplit - 1);
  float m_run = -INFINITY, l_run = 0.0f;  // QK role: this thread's head
  float acc[8];
#pragma unroll
  for (int h = 0; h < 8; ++h) acc[h] = 0.0f;

  for (int64_t c0 = k0; c0 < k1; c0 += kChunk) {
    const int nk = chunk_keys(c0);
    __syncthreads();  // the previous chunk's readers are done
    if (c0 != k0) load_chunk(c0, nk);
#pragma unroll
    for (int x = 0; x < kPer; ++x) {
      const int i = tid + x * kQ8Threads;
      if (i < kWords) {
        (&sm.k[0][0][0])[i] = kv_[0][x];
        (&sm.v[0][0][0])[i] = kv_[1][x];
      }
    }
    __syncthreads();

    // ---- QK: score of (head 8 half + hh, key kk) = sum_j d_j sum_i q8 * q
    {
      // this thread's blocks start dh * 8 / kSplit blocks (34 dwords per 4 blocks) into
      // the row, so every byte position below is a compile-time constant
      constexpr int kBlk = 8 / kSplit;
      const uint32_t *krow = sm.k[half][kk] + dh * (34 * kBlk / 4);
      const float4 *qh4 = reinterpret_cast<const float4 *>(sm.q[8 * half + hh] + 32 * kBlk * dh);
      float s = 0.0f;
#pragma unroll
      for (int jj = 0; jj < kBlk; ++jj) {
        // block: bytes o .. o + 33 past krow (f16 d, then 32 int8), within dwords o/4 .. o/4 + 8
        const int o = 34 * jj;
        uint32_t w[9];
#pragma unroll
        for (int x = 0; x < 9; ++x) w[x] = krow[(o >> 2) + x];
        const float d = h16(w[0], (o >> 1) & 1);
        float part = 0.0f;
#pragma unroll
        for (int i4 = 0; i4 < 8; ++i4) {
          const float4 qv = qh4[8 * jj + i4];
          const float qc[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const int pos = (o & 3) + 2 + 4 * i4 + c;
            const int8_t qb = (int8_t)(w[pos >> 2] >> (8 * (pos & 3)));
            part += (float)qb * qc[c];
          }
        }
        s += part * d;
      }
      if constexpr (kSplit == 2) s += __shfl_xor(s, 1, 32);  // blocks 0-3 + blocks 4-7
      // log2 units, clamped at +-100 nats; keys past the chunk are masked
      float s2 = fminf(fmaxf(s * a.sl2, -kSplitClampL2), kSplitClampL2);
      if (kk >= nk) s2 = -INFINITY;
      float mc = s2;
#pragma unroll
      for (int o = 16; o >= kSplit; o >>= 1) mc = fmaxf(mc, __shfl_xor(mc, o, 32));
      const float m_new = fmaxf(m_run, mc);
      const float alpha = (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      const float p = (s2 == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(s2 - m_new);
      float ps = p;
#pragma unroll
      for (int o = 16; o >= kSplit; o >>= 1) ps += __shfl_xor(ps, o, 32);
      l_run = l_run * alpha + ps;
      m_run = m_new;
      if (dh == 0) {
        sm.p[half][kk][hh] = p;
        if (kk == 0) sm.alpha[half][hh] = alpha;
      }
    }
    __syncthreads();

    // ---- PV: element e = tile_e(t / 16, t % 16) of the 8 heads (thread t holds the
    // partial's tile-order entry t, so that its stores are contiguous across lanes):
    // acc = acc * alpha + sum_k p * (d_j * q8)
    {
      const int e = tile_e(t >> 4, t & 15), j = e >> 5, ob = 34 * j + 2 + (e & 31);
#pragma unroll
      for (int h = 0; h < 8; ++h) acc[h] *= sm.alpha[half][h];
      const int wd = (34 * j) >> 2, hd = ((34 * j) >> 1) & 1, wq = ob >> 2, sq = 8 * (ob & 3);
      const auto pv_key = [&](int key) {
        const uint32_t *vrow = sm.v[half][key];
        const float d = h16(vrow[wd], hd);
        const int8_t qb = (int8_t)(vrow[wq] >> sq);
        const float vv = (float)qb * d;
        const float4 p0 = *reinterpret_cast<const float4 *>(&sm.p[half][key][0]);
        const float4 p1 = *reinterpret_cast<const float4 *>(&sm.p[half][key][4]);
        acc[0] += p0.x * vv;
        acc[1] += p0.y * vv;
        acc[2] += p0.z * vv;
        acc[3] += p0.w * vv;
        acc[4] += p1.x * vv;
        acc[5] += p1.y * vv;
        acc[6] += p1.z * vv;
        acc[7] += p1.w * vv;
      };
      if (nk == kChunk) {  // a full chunk: unrolled, its LDS reads issued ahead
#pragma unroll
        for (int key = 0; key < kChunk; ++key) pv_key(key);
      } else {
        for (int key = 0; key < nk; ++key) pv_key(key);
      }
    }
  }

  // ---- partial of this workgroup (tile order), m and l per head
  float *P = a.part + (int64_t)wg * 16 * kPartRow;
  const int idx = t;  // tile-order entry t (element tile_e(t / 16, t % 16))
#pragma unroll
  for (int h = 0; h < 8; ++h) P[(8 * half + h) * kPartRow + idx] = acc[h];
  if (kk == 0 && dh == 0) a.ml[(int64_t)wg * 16 + 8 * half + hh] = float2{m_run, l_run};
}

// ---- MFMA decode over 32-key blocks (caches up to 32k keys per segment)
//
// A workgroup of 8 waves owns a key range of one segment (kpw keys, a multiple of 32) and
// one KV head: decode workgroup w (after the quantizing ones) serves partial slot w / 2
// and KV head w % 2. Per 32-key block the head's K and V rows are staged in LDS (with
// the d_j of both); wave w builds, in registers, the QK A fragments of tile t = w / 4 and
// blocks j = 2 (w % 4), + 1 (int8 codes, exact in fp16) and the PV B fragments of block
// j = w (its codes, exact in fp16: two 16-column tiles, q8_v_codes_dec). Its QK MFMAs (q
// as B: columns 0-7 the fp16 hi parts of the group's 8 heads, 8-15 the lo remainders,
// converted once per workgroup) are scaled by d_j * scale * log2(e) of their keys in
// f32, and the waves' parts are summed through LDS; the hi and lo columns are summed
// across lanes n and n ^ 8. The softmax weights times the V d_j of their keys enter PV
// as A rows 0-7 (fp16 hi) and 8-15 (lo remainder): one MFMA per tile, rows h and h + 8
// summed at the end. The partial goes out in tile order, as the other decode kernels
// write it, for decode_combine_kernel.
constexpr int kQ8mThreads = 512;
struct Q8mSmem {
  h8 qf[8][64];                      // QK B operands: [block j][lane]
  uint32_t raw[2][32][kQ8RowWords];  // [K / V][key][row]
  float kd[8][32];                   // [block j][key]: K's d_j * sl2 (written when staged)
  float vd[8][32];                   // [block j][key]: V's d_j (written when staged)
  float4 sp[8][64];                  // each wave's part of its tile's scores: [wave][lane]
};

// The MFMA decode is on unless PKV_Q8_MFMA=0 (the VALU kernel, kept for comparison).
static inline bool q8_mfma_enabled() {
  static const bool on = [] {
    const char *e = getenv("PKV_Q8_MFMA");
    return !(e && e[0] == '0');
  }();
  return on;
}

__device__ __forceinline__ float xsum16(float x) {  // x of lanes l and l ^ 16, summed
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}

// PV B fragments of the two tiles x = 0, 1 of block j of a staged 32-key block, the
// codes themselves as fp16 (exact; d_j goes into the weights): column n of tile x is
// element 32 j + 4 (n & 7) + 2 x + (n >> 3), so lane (n, g) reads, for each of keys
// 8 g .. + 7, the one dword holding codes 4 (n & 7) .. + 3 of block j (two bytes past a
// dword boundary for even j) and keeps bytes n >> 3 (tile 0) and 2 + (n >> 3) (tile 1).
// v_perm gathers those bytes of two keys into one dword, which i8x4_to_h4 turns into
// the fp16 pairs of both tiles. Every LDS read is issued before the first wait.
__device__ __forceinline__ void q8_v_codes_dec(const uint32_t (*rows)[kQ8RowWords], int j,
                                               int lane, uint32_t (&wb)[2][4]) {
  const int n = lane & 15, g = lane >> 4;
  const int cb = 34 * j + 2 + 4 * (n & 7), cw = cb >> 2;  // byte / dword of the four codes
  const int sh = cb & 3;  // 0 (odd j: the codes are one dword) or 2 (even j: two)
  uint32_t c0[8], c1[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    c0[k] = rows[8 * g + k][cw];
    c1[k] = sh ? rows[8 * g + k][cw + 1] : 0u;
  }
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t b0 = n >> 3, b1 = 2 + b0;
  const uint32_t sel = b0 | ((4 + b0) << 8) | (b1 << 16) | ((4 + b1) << 24);
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t w0 = __builtin_amdgcn_alignbyte(c1[2 * p], c0[2 * p], sh);
    const uint32_t w1 = __builtin_amdgcn_alignbyte(c1[2 * p + 1], c0[2 * p + 1], sh);
    h2 lo, hi;  // keys 8 g + 2 p, + 1 of tile 0 (lo) and tile 1 (hi)
    i8x4_to_h4(__builtin_amdgcn_perm(w1, w0, sel), lo, hi);
    wb[0][p] = as_u(lo);
    wb[1][p] = as_u(hi);
  }
}

// kOne: a one-segment launch; kFused: the launch appends the new rows. Neither needs a
// kernel argument to tell a workgroup its role. The leading scalar arguments repeat what
// the decode workgroups need first (segment 0's rows and key count, q, the partial
// buffers, the row stride, kpw, sl2): the build preloads them into SGPRs, so the first
// loads of a one-segment launch wait for no kernel-argument fetch.
template <bool kOne, bool kFused>
__global__ __launch_bounds__(kQ8mThreads) void q8_decode_mfma_kernel(
    const uint8_t *k_0, const uint8_t *v_0, const float *q, float *part, float2 *mlb, int rs_t,
    int kpw, int seq_k0, float sl2, Q8Args a) {
  __shared__ Q8mSmem sm;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  // ---- fused append: the first 4 n workgroups quantize new row r = 4 s + 2 p + kv (K
  // p = 0, V p = 1) each; the decode workgroups follow
  const int nq = kFused ? (kOne ? 4 : 4 * a.nseg) : 0;
  const int wg = (int)blockIdx.x - nq, slot = wg >> 1, kv = wg & 1;
  if (kFused && wg < 0) {
    if (tid >= 256) return;
    const int row = wg + nq, rs = row >> 2, p = (row >> 1) & 1, kvr = row & 1;
    const float x = (p ? a.v_new : a.k_new)[((int64_t)rs * 2 + kvr) * 256 + tid];
    const DecodeSeg &rg = a.seg[rs];
    uint8_t *dst = (p ? rg.v : rg.k) + rg.t_new * a.rs_t + kvr * a.rs_h;
    a.dq[(int64_t)row * 256 + tid] = q8_quantize_row_lanes(x, dst, tid);
    return;
  }
  // the segment of this workgroup (segment 0 of a one-segment launch from the scalar
  // arguments)
  const uint8_t *sk = k_0, *sv = v_0;
  int64_t seq_k = seq_k0;
  int wg0 = 0, qi = 0;
  if (!kOne) {
    int b = 0;
    while (b + 1 < a.nseg && slot >= a.seg[b + 1].wg0) ++b;
    const DecodeSeg sg = a.seg[b];
    sk = sg.k;
    sv = sg.v;
    seq_k = sg.seq_k;
    wg0 = sg.wg0;
    qi = sg.qi;
  }
  const int64_t k0 = (int64_t)(slot - wg0) * kpw;
  const int64_t k1 = k0 + kpw < seq_k ? k0 + kpw : seq_k;
  const uint8_t *kbase = sk + kv * kQ8Row, *vbase = sv + kv * kQ8Row;

  // head kv's K and V rows (272 bytes per key) of the block at c0: every load is issued
  // before the first LDS store, unconditionally (pieces past the block and keys past nk
  // read the last piece / key again, and are dropped or stored as 0), so that no load
  // waits for another. The K pieces 2 j (j < 8), whose halfword j is d_j, also store
  // d_j * sl2 for the QK scaling, the V pieces 2 j d_j for the PV operands.
  constexpr int kPieces = 2 * 32 * (kQ8RowB / 16);  // 16-byte pieces of a staged block
  constexpr int kPer = (kPieces + kQ8mThreads - 1) / kQ8mThreads;
  uint4 w[kPer];
  auto load_block = [&](int64_t c0, int nk) {
#pragma unroll
    for (int x = 0; x < kPer; ++x) {
      const int c = min(tid + x * kQ8mThreads, kPieces - 1);
      const int tn = c / (kPieces / 2), r = c % (kPieces / 2);
      const int key = min(r / 17, nk - 1), piece = r % 17;
      w[x] = *reinterpret_cast<const uint4 *>((tn ? vbase : kbase) + (c0 + key) * rs_t + 16 * piece);
    }
  };
  auto store_block = [&](int nk) {
#pragma unroll
    for (int x = 0; x < kPer; ++x) {
      const int c = tid + x * kQ8mThreads;
      const int tn = c / (kPieces / 2), r = c % (kPieces / 2);
      const int key = r / 17, piece = r % 17;
      if (c < kPieces) {
        const uint4 v = key < nk ? w[x] : uint4{0u, 0u, 0u, 0u};
        *reinterpret_cast<uint4 *>(&sm.raw[tn][key][4 * piece]) = v;
        if (piece < 16 && (piece & 1) == 0) {
          const int j = piece >> 1;
          const uint32_t dw = (j >> 1) == 0 ? v.x : (j >> 1) == 1 ? v.y : (j >> 1) == 2 ? v.z : v.w;
          const float d = h2f((j & 1) ? (dw >> 16) : (dw & 0xFFFF));
          if (tn == 0) sm.kd[j][key] = d * sl2;
          else sm.vd[j][key] = d;
        }
      }
    }
  };
  // ---- q of the head group as QK B operands, built once: fragment (j, lane (n, g)) holds
  // elements 32 j + 8 g .. + 7 of head 8 kv + n % 8, as the fp16 hi part (n < 8) or the
  // lo remainder (n >= 8); thread t = 32 j + 8 g + h loads those of head h once and builds
  // both fragments
  {
    const int tq = tid & 255, j = tq >> 5, gq = (tq >> 3) & 3, hq = tq & 7;
    const float *qrow = q + ((int64_t)qi * 16 + 8 * kv + hq) * 256 + 32 * j + 8 * gq;
    const float4 q0 = *reinterpret_cast<const float4 *>(qrow);  // threads >= 256 load again
    const float4 q1 = *reinterpret_cast<const float4 *>(qrow + 4);
    if (k0 < k1) load_block(k0, (int)(k1 - k0 < kBlk ? k1 - k0 : kBlk));
    if (tid < 256) {
      const float v8[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
      h8 fh, fl;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const _Float16 hi = (_Float16)v8[k];
        fh[k] = hi;
        fl[k] = (_Float16)(v8[k] - (float)hi);
      }
      sm.qf[j][16 * gq + hq] = fh;
      sm.qf[j][16 * gq + 8 + hq] = fl;
    }
  }

  const int tw = wv >> 2, qd = wv & 3;  // QK: tile tw, blocks 2 qd, 2 qd + 1
  // PV: block j = wv (two tiles), its d_j folded into the weights
  f4 acc[2];
#pragma unroll
  for (int x = 0; x < 2; ++x) acc[x] = f4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;  // head n % 8 (the same in lanes n, n ^ 8 and every g)

  for (int64_t c0 = k0; c0 < k1; c0 += kBlk) {
    const int nk = (int)(k1 - c0 < kBlk ? k1 - c0 : kBlk);
    if (c0 != k0) {
      __syncthreads();  // the previous block's readers are done
      load_block(c0, nk);
    }
    store_block(nk);
    __syncthreads();
    // ---- QK of tile tw over blocks j = 2 qd, 2 qd + 1, A fragments in registers (lane
    // (r, g): key q8_key(r, tw), elements 32 j + 8 g .. + 7)
    f4 cq[2];
    {
      const h8 qb0 = sm.qf[2 * qd][lane], qb1 = sm.qf[2 * qd + 1][lane];
      const uint32_t *row = &sm.raw[0][q8_key(n, tw)][0];
      const int w0i = (68 * qd + 2 + 8 * g) >> 2;  // block 2 qd: two bytes past w0i
      uint32_t x[5];
#pragma unroll
      for (int i = 0; i < 5; ++i) x[i] = row[w0i + (i < 3 ? i : 6 + i)];  // block 2 qd + 1 at w0i + 9
      __builtin_amdgcn_sched_barrier(0);  // every read above is issued before the first wait
      const uint32_t kw[2][2] = {{__builtin_amdgcn_alignbyte(x[1], x[0], 2),
                                  __builtin_amdgcn_alignbyte(x[2], x[1], 2)},
                                 {x[3], x[4]}};
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        h2 a0, a1, a2, a3;
        i8x4_to_h4(kw[jj][0], a0, a1);
        i8x4_to_h4(kw[jj][1], a2, a3);
        const h8 ka = h8{a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
        cq[jj] = mfma32(ka, jj ? qb1 : qb0, f4{0.f, 0.f, 0.f, 0.f});
      }
    }
    // ---- PV B fragments of this wave's two tiles and the d_j of its keys 8 g .. + 7,
    // in registers (while the MFMAs run)
    uint32_t wb[2][4];
    q8_v_codes_dec(sm.raw[1], wv, lane, wb);
    const float4 vd0 = *reinterpret_cast<const float4 *>(&sm.vd[wv][8 * g]);
    const float4 vd1 = *reinterpret_cast<const float4 *>(&sm.vd[wv][8 * g + 4]);
    // this wave's part of its tile's scores, scaled by its keys' d_j, to LDS
    {
      float4 part = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const float4 dk = *reinterpret_cast<const float4 *>(&sm.kd[2 * qd + jj][8 * g + 4 * tw]);
        part.x = fmaf(dk.x, cq[jj][0], part.x);
        part.y = fmaf(dk.y, cq[jj][1], part.y);
        part.z = fmaf(dk.z, cq[jj][2], part.z);
        part.w = fmaf(dk.w, cq[jj][3], part.w);
      }
      sm.sp[wv][lane] = part;
    }
    __syncthreads();  // every wave's part of the scores is in LDS

    // ---- the scores: sc[4 t + i] of key 8 g + 4 t + i for column n, summed over the
    // waves' blocks in block order (blocks 0-1, 2-3, 4-5, 6-7)
    float sc[8];
    float4 sp8[8];
#pragma unroll
    for (int w2 = 0; w2 < 8; ++w2) sp8[w2] = sm.sp[w2][lane];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float4 tot = sp8[4 * t];
#pragma unroll
      for (int w2 = 1; w2 < 4; ++w2) {
        const float4 pw = sp8[4 * t + w2];
        tot.x += pw.x;
        tot.y += pw.y;
        tot.z += pw.z;
        tot.w += pw.w;
      }
      sc[4 * t + 0] = tot.x;
      sc[4 * t + 1] = tot.y;
      sc[4 * t + 2] = tot.z;
      sc[4 * t + 3] = tot.w;
    }
    // hi + lo columns (lanes n and n ^ 8), clamp, mask the keys past the range
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float s = sc[k] + ror8(sc[k]);
      sc[k] = 8 * g + k < nk ? fminf(fmaxf(s, -kSplitClampL2), kSplitClampL2) : -INFINITY;
    }
    // ---- online softmax of head n % 8 over the block (lanes n, n + 16, n + 32, n + 48)
    float bm = sc[0];
#pragma unroll
    for (int k = 1; k < 8; ++k) bm = fmaxf(bm, sc[k]);
    bm = xmax32(xmax16(bm));
    const float m_new = fmaxf(m_run, bm);
    // some head's max rose after the first block: rescale its sums (rows by head; on the
    // first block they are still 0)
    if (c0 != k0 && __any(m_new != m_run)) {
      const float alpha = (m_new == m_run) ? 1.0f
                          : (m_run == -INFINITY) ? 0.0f
                                                 : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
      // row 4 g + i is head (4 g + i) % 8, whose alpha lane (4 g + i) % 8 holds
      const auto lane_alpha = [&](int k) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), k));
      };
      const bool odd = (g & 1) != 0;
      float ai[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lo = lane_alpha(i), hi = lane_alpha(i + 4);
        ai[i] = odd ? hi : lo;
      }
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[x][i] *= ai[i];
    }
    m_run = m_new;
    float p[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      p[k] = (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(sc[k] - m_run);
      l_run += p[k];
    }
    // A rows: n < 8 the fp16 hi parts of head n's weights times d_j of their keys, n >= 8
    // the lo remainders
    const float dv[8] = {vd0.x, vd0.y, vd0.z, vd0.w, vd1.x, vd1.y, vd1.z, vd1.w};
    uint32_t wa[4];
#pragma unroll
    for (int k2 = 0; k2 < 4; ++k2) {
      const float p0 = p[2 * k2] * dv[2 * k2], p1 = p[2 * k2 + 1] * dv[2 * k2 + 1];
      const uint32_t hw = as_u(h2{(_Float16)p0, (_Float16)p1});
      const uint32_t lw = fp16_sub2(p0, p1, hw);
      wa[k2] = n < 8 ? hw : lw;
    }
    const h8 A = __builtin_bit_cast(h8, u4{wa[0], wa[1], wa[2], wa[3]});
#pragma unroll
    for (int x = 0; x < 2; ++x)
      acc[x] = mfma32(A, __builtin_bit_cast(h8, u4{wb[x][0], wb[x][1], wb[x][2], wb[x][3]}), acc[x]);
  }

  // ---- partial: rows h (hi weights) and h + 8 (lo) summed (lanes g and g + 2); element
  // 32 wv + 4 (n & 7) + 2 x + (n >> 3) of head 8 kv + 4 g + i (lanes 0-31) goes to its
  // tile-order entry (8 consecutive entries per 8 lanes). Agent-scope (write-through)
  // stores: the combine launch reads them from another XCD's L2 misses anyway, and the
  // launch's end then has fewer dirty lines to write back.
  float *P = part + (int64_t)slot * 16 * kPartRow;
  float r[2][4];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int i = 0; i < 4; ++i) r[x][i] = xsum32(acc[x][i]);
  if (g < 2) {
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const int ent = tile_index(32 * wv + 4 * (n & 7) + 2 * x + (n >> 3));
#pragma unroll
      for (int i = 0; i < 4; ++i) store_sc1(P + (8 * kv + 4 * g + i) * kPartRow + ent, r[x][i]);
    }
  }
  // the weights' sum of head n % 8 over the lanes g (each holds its 8 keys)
  float lt = xsum16(l_run);
  lt = xsum32(lt);
  if (wv == 0 && g == 0 && n < 8) {
    float *mlo = reinterpret_cast<float *>(mlb + ((int64_t)slot * 16 + 8 * kv + n));
    store_sc1(mlo, m_run);
    store_sc1(mlo + 1, lt);
  }
}

}  // namespace

// Plan and launch the Q8_0 decode and the combine over n <= kMaxSegs segments.
static int launch_q8_segments(const DecodeSegIn *in, int n, const float *q, const float *k_new,
                              const float *v_new, float *out, int64_t rs_t, int64_t rs_h,
                              float scale, Workspace &ws, hipStream_t s) {
  Q8Args d;
  const bool fused = k_new != nullptr;
  int64_t longest = 0;
  for (int i = 0; i < n; ++i) {
    d.seg[i].k = in[i].k;
    d.seg[i].v = in[i].v;
    d.seg[i].seq_k = fused ? in[i].seq_k - 1 : in[i].seq_k;
    d.seg[i].t_new = in[i].seq_k - 1;
    d.seg[i].nblk = 0;
    d.seg[i].qi = i;
    if (d.seg[i].seq_k > longest) longest = d.seg[i].seq_k;
  }
  d.dseg = nullptr;
  d.wps = 0;
  // The MFMA kernel for caches up to 32768 keys in the standard row layout (both heads'
  // 272-byte rows adjacent, 16-byte aligned): 32-key blocks, one to four per workgroup
  // (up to 256 workgroups per segment). Otherwise the VALU kernel: one chunk per
  // workgroup while that keeps <= 512 partials per segment (16-key chunks up to 8192
  // keys, 32-key chunks beyond), more chunks per workgroup for longer caches.
  bool mfma = longest <= 32768 && rs_h == kQ8Row && rs_t % 16 == 0 && rs_t < (1 << 24) &&
              q8_mfma_enabled();
  for (int i = 0; i < n && mfma; ++i)
    mfma = (reinterpret_cast<uintptr_t>(in[i].k) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(in[i].v) & 15) == 0;
  int64_t kpw;
  int chunk;
  if (mfma) {
    chunk = kBlk;
    kpw = kBlk * ((longest + 256 * kBlk - 1) / (256 * kBlk));
    if (kpw < kBlk) kpw = kBlk;
  } else {
    kpw = (longest + 511) / 512;
    chunk = kpw <= 16 ? 16 : kQ8Chunk;
    kpw = (kpw + chunk - 1) / chunk * chunk;
    if (kpw < chunk) kpw = chunk;
  }
  CombineArgs c;
  int wg = 0;
  for (int i = 0; i < n; ++i) {
    d.seg[i].wg0 = wg;
    c.wg0[i] = wg;
    const int64_t w = d.seg[i].seq_k > 0 ? (d.seg[i].seq_k + kpw - 1) / kpw : 1;
    wg += (int)w;
    c.wg1[i] = wg;
  }
  d.nseg = n;
  d.nwg = wg;
  d.kpw = (int)kpw;
  d.rs_t = rs_t;
  d.rs_h = rs_h;
  d.sl2 = scale * 1.4426950408889634f;
  d.q = q;
  d.k_new = k_new;
  d.v_new = v_new;
  const size_t part_floats = (size_t)wg * 16 * kPartRow, ml_floats = (size_t)wg * 16 * 2;
  const size_t need = (part_floats + ml_floats + (size_t)n * 4 * 256) * sizeof(float);
  int rc = ws.reserve(need);
  if (rc) return rc;
  d.part = static_cast<float *>(ws.ptr);
  d.ml = reinterpret_cast<float2 *>(d.part + part_floats);
  d.dq = d.part + part_floats + ml_floats;
  if (mfma) {  // one workgroup per new row, then two (KV heads) per slot
    d.nwg = 2 * wg;
    const int nq = fused ? 4 * n : 0;
    const dim3 grid((unsigned)(2 * wg + nq)), block(kQ8mThreads);
    auto go = [&](auto kern) {
      hipLaunchKernelGGL(kern, grid, block, 0, s, d.seg[0].k, d.seg[0].v, q, d.part, d.ml,
                         (int)rs_t, d.kpw, (int)d.seg[0].seq_k, d.sl2, d);
    };
    if (n == 1 && fused) go(q8_decode_mfma_kernel<true, true>);
    else if (n == 1) go(q8_decode_mfma_kernel<true, false>);
    else if (fused) go(q8_decode_mfma_kernel<false, true>);
    else go(q8_decode_mfma_kernel<false, false>);
  } else if (chunk == 16) {
    hipLaunchKernelGGL(q8_decode_kernel<16>, dim3((unsigned)wg), dim3(kQ8Threads), 0, s, d);
  } else {
    hipLaunchKernelGGL(q8_decode_kernel<kQ8Chunk>, dim3((unsigned)wg), dim3(kQ8Threads), 0, s,
                       d);
  }
  PKV_HIP(hipGetLastError());
  c.part = d.part;
  c.ml = d.ml;
  c.q = q;
  c.dq = fused ? d.dq : nullptr;
  c.out = out;
  c.sl2 = d.sl2;
  if (const int rc_ = launch_combine(c, n, s)) return rc_;
  return PKV_OK;
}

// Paged decode: every page run is a segment with the same number of workgroups (wps =
// page_tokens / keys per workgroup), so workgroup w serves segment w / wps; the combine
// merges all partials of a sequence (its segments are consecutive). Up to kMaxSegs
// segments travel in the kernel arguments; more go to a device table in the workspace.
int launch_paged_decode_q8(const PagedSeg *segs, int nseg, int nseq, int page_tokens,
                           const float *q, float *out, int64_t rs_t, int64_t rs_h, float scale,
                           void *stage, Workspace &ws, hipStream_t s) {
  static_assert(sizeof(DecodeSeg) <= kPagedSegBytes, "segment table entry size");
  static_assert(kPagedArgSegs == kMaxSegs, "kernel-argument segment count");
  if (nseq < 1 || nseq > kMaxPagedSeqs || nseg < nseq || page_tokens % kQ8Chunk != 0)
    return set_error(PKV_ERR_ARG, "paged decode: bad segment plan");
  if (rs_h != kQ8Row || !decode_rows_fit(page_tokens, rs_t)) return PKV_ERR_UNSUPPORTED;
  // keys per workgroup: a multiple of 32 dividing the page into equal parts, aiming at
  // about 768 workgroups over the whole launch
  int64_t kpw = (int64_t)page_tokens * nseg / 768;
  kpw = (kpw + kQ8Chunk - 1) / kQ8Chunk * kQ8Chunk;
  if (kpw < kQ8Chunk) kpw = kQ8Chunk;
  if (kpw > page_tokens) kpw = page_tokens;
  const int wps = (int)((page_tokens + kpw - 1) / kpw);
  const int64_t nwg64 = (int64_t)nseg * wps;
  if (nwg64 > (1 << 24)) return set_error(PKV_ERR_ARG, "paged decode: too many pages");
  const int nwg = (int)nwg64;
  std::vector<DecodeSeg> tab((size_t)nseg);
  CombineArgs c;
  int qprev = -1;
  for (int i = 0; i < nseg; ++i) {
    DecodeSeg &d = tab[(size_t)i];
    if (segs[i].qi < qprev || segs[i].qi >= nseq || segs[i].len < 0 || segs[i].len > page_tokens)
      return set_error(PKV_ERR_ARG, "paged decode: segments out of order");
    while (qprev < segs[i].qi) c.wg0[++qprev] = i * wps;
    c.wg1[qprev] = (i + 1) * wps;
    d.k = segs[i].k;
    d.v = segs[i].v;
    d.seq_k = segs[i].len;
    d.t_new = 0;
    d.nblk = 0;
    d.wg0 = i * wps;
    d.qi = segs[i].qi;
    d.voff = 0;
  }
  if (qprev != nseq - 1) return set_error(PKV_ERR_ARG, "paged decode: a sequence has no page");
  Q8Args d;
  d.nseg = nseg;
  d.nwg = nwg;
  d.kpw = (int)kpw;
  d.rs_t = rs_t;
  d.rs_h = rs_h;
  d.sl2 = scale * 1.4426950408889634f;
  d.q = q;
  d.k_new = d.v_new = nullptr;
  const size_t part_floats = (size_t)nwg * 16 * kPartRow, ml_floats = (size_t)nwg * 16 * 2;
  const size_t tab_off = (part_floats + ml_floats) * sizeof(float);
  const size_t tab_bytes = nseg > kMaxSegs ? (size_t)nseg * sizeof(DecodeSeg) : 0;
  int rc = ws.reserve(tab_off + tab_bytes);
  if (rc) return rc;
  d.part = static_cast<float *>(ws.ptr);
  d.ml = reinterpret_cast<float2 *>(d.part + part_floats);
  d.dq = nullptr;
  d.wps = wps;
  if (nseg <= kMaxSegs) {
    for (int i = 0; i < nseg; ++i) d.seg[i] = tab[(size_t)i];
    d.dseg = nullptr;
  } else {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    PKV_HIP(hipStreamIsCapturing(s, &cap));
    if (cap != hipStreamCaptureStatusNone)
      return set_error(PKV_ERR_UNSUPPORTED,
                       "paged decode over more than 32 pages cannot be captured in a graph");
    if (stage == nullptr) return set_error(PKV_ERR_ARG, "paged decode: no staging buffer");
    memcpy(stage, tab.data(), tab_bytes);
    DecodeSeg *dtab = reinterpret_cast<DecodeSeg *>(static_cast<uint8_t *>(ws.ptr) + tab_off);
    PKV_HIP(hipMemcpyAsync(dtab, stage, tab_bytes, hipMemcpyHostToDevice, s));
    d.dseg = dtab;
  }
  hipLaunchKernelGGL(q8_decode_kernel<kQ8Chunk>, dim3((unsigned)nwg), dim3(kQ8Threads), 0, s,
                     d);
  PKV_HIP(hipGetLastError());
  c.part = d.part;
  c.ml = d.ml;
  c.q = q;
  c.dq = nullptr;
  c.out = out;
  c.sl2 = d.sl2;
  if (const int rc_ = launch_combine(c, nseq, s)) return rc_;
  return PKV_OK;
}

int launch_attend_q8(const AttnArgs &a, const float *k_new, const float *v_new, uint8_t *kc,
                     uint8_t *vc, int64_t t_new, Workspace &ws, hipStream_t s) {
  if (a.quant != PKV_QUANT_Q8_0 || a.head_dim != 256 || a.num_heads != 16 ||
      a.num_kv_heads != 2 || a.l != 1)
    return PKV_ERR_UNSUPPORTED;
  if (a.causal && a.q_offset + 1 < a.seq_k) return PKV_ERR_UNSUPPORTED;
  const bool fused = k_new != nullptr;
  if (fused && (kc != a.k || vc != a.v || t_new != a.seq_k - 1)) return PKV_ERR_UNSUPPORTED;
  if (a.rs.h != kQ8Row || !decode_rows_fit(a.seq_k, a.rs.t)) return PKV_ERR_UNSUPPORTED;
  for (int b0 = 0; b0 < a.batch; b0 += kMaxSegs) {
    const int nb = a.batch - b0 < kMaxSegs ? a.batch - b0 : kMaxSegs;
    DecodeSegIn in[kMaxSegs];
    for (int i = 0; i < nb; ++i) {
      in[i].k = const_cast<uint8_t *>(a.k) + (int64_t)(b0 + i) * a.rs.b;
      in[i].v = const_cast<uint8_t *>(a.v) + (int64_t)(b0 + i) * a.rs.b;
      in[i].seq_k = a.seq_k;
    }
    const int64_t qo = (int64_t)b0 * 16 * 256, ko = (int64_t)b0 * 2 * 256;
    const int rc = launch_q8_segments(in, nb, a.q + qo, fused ? k_new + ko : nullptr,
                                      fused ? v_new + ko : nullptr, a.out + qo, a.rs.t, a.rs.h,
                                      a.scale, ws, s);
    if (rc) return rc;
  }
  return PKV_OK;
}

int launch_append_attend_batched_q8(int quant, const SeqDesc *seqs, int n, const float *k,
                                    const float *v, const float *q, int num_heads,
                                    int num_kv_heads, int head_dim, float scale, float *out,
                                    Workspace &ws, hipStream_t s) {
  if (quant != PKV_QUANT_Q8_0 || head_dim != 256 || num_heads != 16 || num_kv_heads != 2)
    return PKV_ERR_UNSUPPORTED;
  const int64_t rs_t = 2 * kQ8Row, rs_h = kQ8Row;
  for (int i = 0; i < n; ++i)
    if (seqs[i].len < 1 || !decode_rows_fit(seqs[i].len, rs_t)) return PKV_ERR_UNSUPPORTED;
  for (int b0 = 0; b0 < n; b0 += kMaxSegs) {
    const int nb = n - b0 < kMaxSegs ? n - b0 : kMaxSegs;
    DecodeSegIn in[kMaxSegs];
    for (int i = 0; i < nb; ++i) {
      in[i].k = seqs[b0 + i].k;
      in[i].v = seqs[b0 + i].v;
      in[i].seq_k = seqs[b0 + i].len;
    }
    const int64_t qo = (int64_t)b0 * 16 * 256, ko = (int64_t)b0 * 2 * 256;
    const int rc = launch_q8_segments(in, nb, q + qo, k + ko, v + ko, out + qo, rs_t, rs_h,
                                      scale, ws, s);
    if (rc) return rc;
  }
  return PKV_OK;
}

}  // namespace pkv
