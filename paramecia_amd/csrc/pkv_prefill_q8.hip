// MFMA prefill-chunk attention over a Q8_0 cache for the Qwen3-Next full-attention shape
// (16 query heads, 2 KV heads, head_dim 256), gfx950.
//
// Role: the reference's flash_attn_q8 with seq_q > 1 (paramecia-model/src/ops.rs:756-792,
// called at qwen3_next.rs:2531-2561 with q_offset = seq_k - l for every prefill chunk of
// a Q8_0 cache, the serving backend's default, paramecia-llm/src/backend/local.rs:111-115)
// and the CPU SDPA it replaces (qwen3_next.rs:2580-2605): the chunk's l queries attend
// causally over every key (query i sees key j iff j <= i + q_offset), GQA group 8,
// scores scaled, clamped to +-100, soft-maxed and applied to V. A Q8_0 row is 8 blocks
// of {f16 d, 32 x int8}: element e is int8 * d of block e / 32 (BlockQ8_0::to_float).
//
// Work split (as the Q4K prefill kernel): a workgroup owns one KV head, 16 query
// positions (128 rows = 16 positions x 8 heads of the group, 16 rows per wave) and one
// split of the keys. Every 32-key block is staged raw in LDS by waves 6 and 7 (nine
// 16-byte loads per tensor, lane-addressed) and dequantized ONCE into fp16 MFMA operand
// fragments in LDS - K by waves 0-1, V by waves 2-5 - which all eight waves then
// consume, so the dequantization is shared by 128 query rows. (Wave w runs on SIMD w % 4:
// each SIMD holds one K or V dequantizing wave and one more.)
//
// Arithmetic (exact fp16 operands or hi + lo pairs, f32 accumulation):
//   QK: per Q8 block j (32 elements, one MFMA K step), A[key][e] = int8 codes (exact in
//       fp16), B[e][row] = q as fp16 hi and lo parts (two MFMAs into one accumulator);
//       the block's sum times d_j * scale * log2(e) of its key is added in f32.
//   PV: B[key][e] = int8 * d (at most 18 significant bits) as an fp16 hi part and the
//       exact lo remainder, A[row][key] = p as fp16 hi and lo parts: hi*hi + lo*hi +
//       hi*lo in f32 (the dropped lo*lo is 2^-22 of a term). One fp16 rounding of V
//       would put row errors near 3e-4 of the row. The output columns are in the
//       decode kernels' tile order (column n of tile T is element tile_e(T, n)), so that
//       a lane's four consecutive codes of one block feed four tiles.
// Keys are permuted inside a block so that the QK result layout equals the PV
// A-operand layout (lane (n, g) holds keys 8g..8g+7 of row n): the scores never leave
// registers.
#include "pkv_mfma_common.hpp"
#include "pkv_prefill_common.hpp"
#include "pkv_q8_common.hpp"

namespace pkv {

namespace {

constexpr int kQ8Loads = 9;         // 16-byte loads per lane per tensor and block
constexpr int kQ8StageB = 9216;     // 32 rows (8704 B) + the last load's overrun
static_assert(kQ8Loads * 64 * 16 == kQ8StageB && 32 * kQ8RowB <= kQ8StageB, "stage size");

struct Q8Raw {
  uint8_t k[kQ8StageB], v[kQ8StageB];
};
// fp16 operand fragments and the K scale table of one 32-key block of one KV head
struct Q8Dq {
  h8 ka[2][8][64];            // QK A: [tile][Q8 block j][lane]
  float kd[8][kBlk];          // d_j * scale * log2(e) per key
  h8 vh[16][64], vl[16][64];  // PV B hi / lo: [tile][lane]
};
struct Q8PfSmem {
  Q8Raw raw[kRaw];
  Q8Dq dq[2];  // block i's operands in dq[i & 1] while block i + 1's are built
};
static_assert(sizeof(Q8PfSmem) <= 160 * 1024, "LDS budget of one workgroup");

// Waves 0-1: the QK A fragments of tile t: lane (r, g) takes key q8_key(r, t), elements
// 32 j + 8 g .. + 7 of every block j; lanes g = 0 also store the key's d_j * sl2.
__device__ __forceinline__ void q8_dq_keys(const Q8Raw &st, Q8Dq &D, float sl2, int t, int lane) {
  const int r = lane & 15, g = lane >> 4;
  const int kk = q8_key(r, t);
  const uint32_t *row = reinterpret_cast<const uint32_t *>(st.k + kk * kQ8RowB);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    // codes at byte 34 j + 2 + 8 g of the row: dword aligned for odd j, two bytes past a
    // dword for even j
    const int b0 = 34 * j + 2 + 8 * g;
    uint32_t w0, w1;
    if (j & 1) {
      w0 = row[b0 >> 2];
      w1 = row[(b0 >> 2) + 1];
    } else {
      const uint32_t x0 = row[b0 >> 2], x1 = row[(b0 >> 2) + 1], x2 = row[(b0 >> 2) + 2];
      w0 = __builtin_amdgcn_alignbyte(x1, x0, 2);
      w1 = __builtin_amdgcn_alignbyte(x2, x1, 2);
    }
    h2 a0, a1, a2, a3;
    i8x4_to_h4(w0, a0, a1);
    i8x4_to_h4(w1, a2, a3);
    D.ka[t][j][lane] = h8{a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
    if (g == 0) {
      const uint32_t dw = row[(34 * j) >> 2];  // d: the low half for even j, the high for odd
      D.kd[j][kk] = h2f((j & 1) ? (dw >> 16) : (dw & 0xFFFF)) * sl2;
    }
  }
}

// Waves 2-5 (vw = 0..3): the PV B fragments of unit vw (q8_v_words), into LDS.
template <int kHl>
__device__ __forceinline__ void q8_dq_values(const Q8Raw &st, Q8Dq &D, int h, int lane) {
  uint32_t wh[4][4], wl[4][4];
  q8_v_words<kHl>(reinterpret_cast<const uint32_t *>(st.v), kQ8RowB / 4, h, lane, wh, wl);
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int T = 8 * h + kHl + 2 * b;
    D.vh[T][lane] = __builtin_bit_cast(h8, u4{wh[b][0], wh[b][1], wh[b][2], wh[b][3]});
    D.vl[T][lane] = __builtin_bit_cast(h8, u4{wl[b][0], wl[b][1], wl[b][2], wl[b][3]});
  }
}

// Per-lane byte offsets of the nine 16-byte loads of one tensor of a block: load i, lane
// l moves 16-byte piece c % 17 of block row c / 17 (c = 64 i + l) to LDS byte 16 c, so
// the rows land contiguous (row R at 272 R). Lanes past the 32 rows (c >= 544) read the
// start of the next block's rows into the stage's tail, which nothing reads.
struct Q8Plan {
  uint32_t off[kQ8Loads];
};
__device__ __forceinline__ Q8Plan make_q8_plan(int lane, uint32_t rs_t) {
  Q8Plan P;
#pragma unroll
  for (int i = 0; i < kQ8Loads; ++i) {
    const int c = 64 * i + lane;
    P.off[i] = (uint32_t)(c / 17) * rs_t + 16u * (uint32_t)(c % 17);
  }
  return P;
}
// The nine loads of one tensor of one block: issued by one wave, so that its vmcnt
// counts exactly its own loads.
__device__ __forceinline__ void issue_q8_tensor(uint8_t *dst, const Q8Plan &P, u4s rsrc,
                                                uint32_t boff) {
  const uint32_t d0 = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)((PKV_LDS void *)dst));
  uint32_t saved;
  asm volatile(
      "s_nop 4\n\t"  // VALU-written SGPRs (v_readfirstlane) read by VMEM: 5 wait states
      "s_mov_b32 %[sv], m0\n\t"
      "s_mov_b32 m0, %[d0]\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o0], %[rs], 0 offen lds\n\t"
      "s_add_u32 m0, %[d0], 0x400\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o1], %[rs], 0 offen lds\n\t"
      "s_add_u32 m0, %[d0], 0x800\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o2], %[rs], 0 offen lds\n\t"
      "s_add_u32 m0, %[d0], 0xc00\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o3], %[rs], 0 offen lds\n\t"
      "s_add_u32 m0, %[d0], 0x1000\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o4], %[rs], 0 offen lds\n\t"
      "s_add_u32 m0, %[d0], 0x1400\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o5], %[rs], 0 offen lds\n\t"
      "s_add_u32 m0, %[d0], 0x1800\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o6], %[rs], 0 offen lds\n\t"
      "s_add_u32 m0, %[d0], 0x1c00\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o7], %[rs], 0 offen lds\n\t"
      "s_add_u32 m0, %[d0], 0x2000\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o8], %[rs], 0 offen lds\n\t"
      "s_mov_b32 m0, %[sv]"
      : [sv] "=&s"(saved)
      : [d0] "s"(d0), [o0] "v"(P.off[0] + boff), [o1] "v"(P.off[1] + boff),
        [o2] "v"(P.off[2] + boff), [o3] "v"(P.off[3] + boff), [o4] "v"(P.off[4] + boff),
        [o5] "v"(P.off[5] + boff), [o6] "v"(P.off[6] + boff), [o7] "v"(P.off[7] + boff),
        [o8] "v"(P.off[8] + boff), [rs] "s"(rsrc)
      : "memory", "scc");
}

__global__ __launch_bounds__(kPfThreads) void q8_prefill_kernel(PrefillArgs a) {
  __shared__ Q8PfSmem sm;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const PfWork wk = prefill_work(a);
  const int tile = wk.tile, kvg = wk.kvg, split = wk.split, b = wk.b;
  const int p0 = tile * kPosPerWG;
  const int pw = p0 + 2 * wave;  // this wave's first position; row n -> pw + n / 8

  // ---- key blocks of this workgroup: its split, cut at the last key any of its queries
  // may see
  int64_t kend = a.seq_k;
  if (a.causal) {
    const int64_t plast = (p0 + kPosPerWG - 1 < a.l ? p0 + kPosPerWG - 1 : a.l - 1);
    const int64_t lim = plast + a.q_offset + 1;
    if (lim < kend) kend = lim;
  }
  const int nblk_all = (int)((kend + kBlk - 1) / kBlk);
  const int kb0 = split * a.bps;
  const int kb1 = kb0 + a.bps < nblk_all ? kb0 + a.bps : nblk_all;
  const int nb = kb1 > kb0 ? kb1 - kb0 : 0;

  const uint8_t *kbase = a.k + b * a.rs_b + kvg * a.rs_h;
  const uint8_t *vbase = a.v + b * a.rs_b + kvg * a.rs_h;
  const uint32_t rs_t = (uint32_t)a.rs_t;
  // rows of keys [0, seq_k) of this head; loads past them return zeros
  const uint32_t span = a.seq_k > 0 ? (uint32_t)(a.seq_k - 1) * rs_t + (uint32_t)kQ8RowB : 0u;
  const u4s rk = make_rsrc(kbase, span), rv = make_rsrc(vbase, span);
  const Q8Plan P = make_q8_plan(lane, rs_t);
  const uint32_t bbytes = kBlk * rs_t;
  const bool loader = wave >= 6;
  auto issue = [&](int i) {  // raw block i of this workgroup into stage i % kRaw
    if (wave == 6) issue_q8_tensor(sm.raw[i % kRaw].k, P, rk, (uint32_t)(kb0 + i) * bbytes);
    if (wave == 7) issue_q8_tensor(sm.raw[i % kRaw].v, P, rv, (uint32_t)(kb0 + i) * bbytes);
  };
  if (loader) {
    if (nb > 0) issue(0);
    if (nb > 1) issue(1);
  }

  // ---- q operands of this wave's 16 rows (row n: position pw + n / 8, head 8 kvg + n % 8):
  // lane (n, g) holds elements 32 j + 8 g .. + 7 for block j, as fp16 hi and lo parts
  h8 qbh[8], qbl[8];
  {
    const int pos = pw + (n >> 3);
    const bool ok = pos < a.l;
    const float *qrow = a.q + (((int64_t)b * a.l + (ok ? pos : 0)) * 16 + 8 * kvg + (n & 7)) * 256 + 8 * g;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      // rows past the chunk read position 0 and are never stored
      const float4 r0 = *reinterpret_cast<const float4 *>(qrow + 32 * j);
      const float4 r1 = *reinterpret_cast<const float4 *>(qrow + 32 * j + 4);
      const float v8[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const _Float16 hi = (_Float16)v8[k];
        qbh[j][k] = hi;
        qbl[j][k] = (_Float16)(v8[k] - (float)hi);
      }
    }
  }

  f4 acc[16];
#pragma unroll
  for (int T = 0; T < 16; ++T) acc[T] = f4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, lsum = 0.0f;
  // position of this lane's row (n): the causal limit of its keys
  const int64_t myq = (int64_t)pw + (n >> 3);
  const int64_t klim = a.causal ? myq + a.q_offset : (int64_t)1 << 62;

  // Waves 0-5 build the fp16 operands of block i + 1 while every wave runs the
  // MFMAs of block i: one barrier per block. Raw stages rotate over kRaw = 3 (blocks
  // i + 1 and i + 2 in flight or landed while block i + 3 is issued).
  auto dequant = [&](int blk) {
    const Q8Raw &st = sm.raw[blk % kRaw];
    Q8Dq &Dn = sm.dq[blk & 1];
    if (wave < 2)
      q8_dq_keys(st, Dn, a.sl2, wave, lane);
    else if (wave < 6) {
      const int vw = __builtin_amdgcn_readfirstlane(wave - 2);
      if (vw & 1)
        q8_dq_values<1>(st, Dn, vw >> 1, lane);
      else
        q8_dq_values<0>(st, Dn, vw >> 1, lane);
    }
  };
  if (nb > 0) {
    if (loader) {  // block 0 landed (block 1 may still fly)
      if (nb > 1)
        asm volatile("s_waitcnt vmcnt(9)" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    if (loader && nb > 2) issue(2);
    dequant(0);
  }
  static_assert(kQ8Loads == 9, "the vmcnt waits count one tensor's loads");
  // Waves 4 and 5 share SIMDs 0 and 1 with waves 0 and 1, which also dequantize: they
  // build block i + 1's operands after block i's MFMAs instead of before, so that on each
  // SIMD one wave's dequantization meets the other's MFMAs.
  const bool late = wave == 4 || wave == 5;
  for (int i = 0; i < nb; ++i) {
    if (loader && i + 1 < nb) {  // block i + 1 landed (block i + 2 may still fly)
      if (i + 2 < nb)
        asm volatile("s_waitcnt vmcnt(9)" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    // operands of block i ready; raw block i + 1 visible; block i - 1's operands and
    // block i's raw stage no longer read
    __syncthreads();
    if (loader && i + 3 < nb) issue(i + 3);
    if (i + 1 < nb && !late) dequant(i + 1);
    const Q8Dq &D = sm.dq[i & 1];

    // ---- QK (two tiles of 16 keys); keys of the block at or past nlim are masked (past
    // the cache, or past this row's causal limit)
    const int64_t key0 = (int64_t)(kb0 + i) * kBlk;
    int64_t lim = a.seq_k < klim + 1 ? a.seq_k : klim + 1;
    lim -= key0;
    const int nlim = lim < 0 ? 0 : (lim > kBlk ? kBlk : (int)lim);
    float sc8[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) sc8[k] = 0.0f;
    // sixteen independent (tile, block) chains of two MFMAs, each then scaled by its keys' d
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const h8 A = D.ka[t][j][lane];
        f4 c = mfma32(A, qbh[j], f4{0.f, 0.f, 0.f, 0.f});
        c = mfma32(A, qbl[j], c);
        const float4 dk = *reinterpret_cast<const float4 *>(&D.kd[j][8 * g + 4 * t]);
        sc8[4 * t + 0] = fmaf(dk.x, c[0], sc8[4 * t + 0]);
        sc8[4 * t + 1] = fmaf(dk.y, c[1], sc8[4 * t + 1]);
        sc8[4 * t + 2] = fmaf(dk.z, c[2], sc8[4 * t + 2]);
        sc8[4 * t + 3] = fmaf(dk.w, c[3], sc8[4 * t + 3]);
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float sc = fminf(fmaxf(sc8[k], -kClampL2), kClampL2);
      sc8[k] = 8 * g + k < nlim ? sc : -INFINITY;
    }
    // ---- online softmax per row (lanes n, n+16, n+32, n+48 hold row n's 32 keys)
    float bm = sc8[0];
#pragma unroll
    for (int k = 1; k < 8; ++k) bm = fmaxf(bm, sc8[k]);
    bm = xmax32(xmax16(bm));
    if (__any(bm > m_run + kPfLazy)) {
      const float m_new = fmaxf(m_run, bm);
      const float alpha = (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      lsum *= alpha;
      m_run = m_new;
      float ai[4];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) ai[ii] = __shfl(alpha, 4 * g + ii);  // rows 4g+ii
#pragma unroll
      for (int T = 0; T < 16; ++T)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) acc[T][ii] *= ai[ii];
    }
    float p[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      // a row with no visible key so far keeps m_run = -inf: its p are 0
      p[k] = (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(sc8[k] - m_run);
      lsum += p[k];
    }
    // ---- PV: A rows = query rows, keys 8g..8g+7, p as fp16 hi and lo parts
    uint32_t wa[4], wl[4];
#pragma unroll
    for (int k2 = 0; k2 < 4; ++k2) {
      wa[k2] = as_u(h2{(_Float16)p[2 * k2], (_Float16)p[2 * k2 + 1]});
      wl[k2] = fp16_sub2(p[2 * k2], p[2 * k2 + 1], wa[k2]);
    }
    const h8 A = __builtin_bit_cast(h8, u4{wa[0], wa[1], wa[2], wa[3]});
    const h8 Al = __builtin_bit_cast(h8, u4{wl[0], wl[1], wl[2], wl[3]});
#pragma unroll
    for (int T = 0; T < 16; ++T) {
      const h8 Bh = D.vh[T][lane], Bl = D.vl[T][lane];
      acc[T] = mfma32(A, Bh, acc[T]);
      acc[T] = mfma32(Al, Bh, acc[T]);
      acc[T] = mfma32(A, Bl, acc[T]);
    }
    if (i + 1 < nb && late) dequant(i + 1);
  }

  // ---- epilogue: row sums, then the output or the split's partial
  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
  float lrow[4], mrow[4];
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) {  // m and l of row 4g+ii live in lane 4g+ii (any g)
    lrow[ii] = __shfl(lsum, 4 * g + ii);
    mrow[ii] = __shfl(m_run, 4 * g + ii);
  }
  if (a.nsplit == 1) {
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int row = 4 * g + ii;
      const int pos = pw + (row >> 3);
      if (pos >= a.l) continue;
      float *orow = a.out + (((int64_t)b * a.l + pos) * 16 + 8 * kvg + (row & 7)) * 256;
      const float inv = lrow[ii] > 0.0f ? 1.0f / lrow[ii] : 0.0f;
#pragma unroll
      for (int T = 0; T < 16; ++T) orow[tile_e(T, n)] = acc[T][ii] * inv;
    }
  } else {
    float *pz = a.part + (((int64_t)(b * a.nsplit + split) * 2 + kvg) * a.l * 8) * 258;
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int row = 4 * g + ii;
      const int pos = pw + (row >> 3);
      if (pos >= a.l) continue;
      float *prow = pz + ((int64_t)pos * 8 + (row & 7)) * 258;
#pragma unroll
      for (int T = 0; T < 16; ++T) prow[16 * T + n] = acc[T][ii];
      if (n == 0) {
        prow[256] = mrow[ii];
        prow[257] = lrow[ii];
      }
    }
  }
}

}  // namespace

int launch_prefill_q8_mfma(const AttnArgs &a, Workspace &ws, hipStream_t s) {
  if (a.quant != PKV_QUANT_Q8_0 || a.head_dim != 256 || a.num_heads != 16 ||
      a.num_kv_heads != 2 || a.l < 2)
    return PKV_ERR_UNSUPPORTED;
  // 16-byte aligned rows of the standard layout, 32-bit offsets within a KV head's rows
  if (a.rs.h != kQ8RowB || (a.rs.t & 15) != 0 || (a.rs.b & 15) != 0 || a.rs.t >= (1 << 24) ||
      a.seq_k >= (1 << 24) || (uint64_t)(a.seq_k + 32) * (uint64_t)a.rs.t >= (1ull << 32) ||
      (reinterpret_cast<uintptr_t>(a.k) & 15) != 0 || (reinterpret_cast<uintptr_t>(a.v) & 15) != 0)
    return PKV_ERR_UNSUPPORTED;
  PrefillArgs d;
  const int rc = prefill_plan(a, a.scale * kLog2e, ws, d);
  if (rc) return rc;
  hipLaunchKernelGGL(q8_prefill_kernel, dim3((unsigned)(d.ntiles * d.ngroups)),
                     dim3(kPfThreads), 0, s, d);
  PKV_HIP(hipGetLastError());
  return prefill_merge(d, a.batch, s);
}

}  // namespace pkv
