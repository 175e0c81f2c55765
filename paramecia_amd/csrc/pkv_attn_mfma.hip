// MFMA decode attention over a Q4K cache for the Qwen3-Next full-attention shape
// (16 query heads, 2 KV heads, head_dim 256), gfx950.
//
// Role: the dequant-fused attention of the reference's flash_attn_q8 path
// (paramecia-model/src/ops.rs:756-792, called at qwen3_next.rs:2531-2561) and the CPU
// SDPA it falls back to (qwen3_next.rs:2580-2605), for a decode step (one query).
//
// Work split: split-K over 32-key blocks. A workgroup (8 waves) owns a contiguous
// block range; waves 0-3 handle KV head 0 and waves 4-7 KV head 1 of the same
// blocks, so the two waves reading the interleaved K/V rows of a token (288 bytes)
// run side by side on one CU. The last workgroup owns the final block and, for a
// fused decode step, first quantizes the new token's rows (bit-exact Q4K).
//
// Arithmetic (per KV head, per 16 keys, MFMA f32_16x16x32_f16):
//   QK: A[key][e] = nibble * sub-block scale code, an integer <= 945 built exactly in
//       fp16 from the packed byte with the 1024-offset trick and one v_pk_fma;
//       B[e][col] = q split into fp16 hi/lo parts: columns 0-7 are the hi parts of the
//       group's 8 heads, 8-15 the lo parts, so hi+lo recover q to ~22 bits.
//       score = d * S1 - dmin * S2 with S2 = sum_j m_j * qsum_j (a 16x16x16 MFMA).
//   PV: B[key][e] = nibble * scale code * 2^e_d (exact fp16, e_d = exponent of d),
//       A[head][key] = p * mantissa(d) in fp16; rows 8-15 of A carry p * mantissa(dmin)
//       and feed the min-term MFMA against B'[key][j] = m_j * 2^e_dmin.
//   All accumulation is f32. Softmax runs in base 2 with the 1/sqrt(d) scale folded
//   in, scores clamped to [-100, 100] (in natural-log units) as the reference does.
#include "pkv_internal.hpp"
#include "pkv_scalar.hpp"
#include "pkv_q4k_lanes.hpp"

namespace pkv {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // 4 waves: 2 per KV head, one wave per SIMD
constexpr int kBlk = 32;
constexpr int kMainWGs = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kClampL2 = 100.0f * 1.4426950408889634f;  // +-100 nats in log2 units

struct DecodeArgs {
  const float *q;  // [B][16][256]
  const uint8_t *k, *v;
  uint8_t *kw, *vw;
  int64_t rs_b, rs_t, rs_h;
  int64_t seq_k;  // keys held in the cache before this step's append (all attended)
  int nblk, nwg_main, bpw;
  float sl2;  // scale * log2(e)
  const float *k_new, *v_new;  // [B][2][256] or null (fused decode step)
  int64_t t_new;
  float *part;  // [B][nwg_main][16][258]
  float *dq;    // [B][4][256] dequantized new rows (K kv0, K kv1, V kv0, V kv1)
};

// Per-wave tables rebuilt for every 32-key block.
struct WaveTab {
  float kd[kBlk], kdm[kBlk];                     // K: d*sl2, dmin*sl2
  float vmd[kBlk], vmdm[kBlk];                   // V: mantissas of d and dmin
  _Float16 vsc[8][kBlk], vc[8][kBlk], vm[8][kBlk];  // V: fp16 constants [j][key]
};

struct Stage;
struct Smem {
  union {
    struct {
      h8 qb[2][8][64];  // QK B operands [kv][step][lane]
      h4 q2[2][64];     // S2 B operands [kv][lane]
      float qf[16][256];  // q staged before the operands are built
      float qs[16][8];    // per head, per 32-element sub-block sums of q
    } qsetup;
    struct {
      WaveTab tab[4];
      char stages[4 * 3 * 2 * 320 * 16];  // Stage[wave][kStages]
    } run;
    struct {
      float o[2][8][256];  // the second wave of each KV head
      float m[2][8], l[2][8];
      float cmin[4][8][8];  // per wave [head][j]
    } merge;
    Q4kScratch quant;
  };
};

__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t o) {
  return (x & m) | o;
}
// Constants kept in VGPRs so that (x & mask) | magic is a single v_and_or_b32 (gfx9
// VOP3 encodings take no literal operands).
__device__ __forceinline__ uint32_t vconst(uint32_t c) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(c));
  return r;
}
struct Masks {
  uint32_t lo, hi, magic;
};
__device__ __forceinline__ h2 as_h2(uint32_t x) { return __builtin_bit_cast(h2, x); }
__device__ __forceinline__ uint32_t as_u(h2 x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ h2 pk_fma(h2 a, h2 b, h2 c) { return __builtin_elementwise_fma(a, b, c); }
__device__ __forceinline__ float ror8(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x128,
                                                            0xF, 0xF, false));
}
__device__ __forceinline__ f4 mfma32(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma16(h4 a, h4 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// 6-bit scale code and min code of sub-block j from the 12 packed bytes (s0 = bytes
// 0-3, s1 = 4-7, s2 = 8-11), get_scale_min_k4.
__device__ __forceinline__ void scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j,
                                          uint32_t &sc, uint32_t &m) {
  const int sh = 8 * (j & 3);
  const uint32_t b_lo = (s0 >> sh) & 0xFF;   // byte j (j < 4) or j-4
  const uint32_t b_mid = (s1 >> sh) & 0xFF;  // byte j+4 (j < 4) or j
  const uint32_t b_hi = (s2 >> sh) & 0xFF;   // byte j+4 (j >= 4)
  const uint32_t sc_lo = b_lo & 63, m_lo = b_mid & 63;
  const uint32_t sc_hi = (b_hi & 0xF) | ((b_lo >> 6) << 4);
  const uint32_t m_hi = (b_hi >> 4) | ((b_mid >> 6) << 4);
  sc = j < 4 ? sc_lo : sc_hi;
  m = j < 4 ? m_lo : m_hi;
}

// exact f16 -> f32 (hardware conversion)
__device__ __forceinline__ float h2f(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// exponent e in [-20, 0] and mantissa d * 2^-e of a non-negative f16 scale
__device__ __forceinline__ void split_scale(float d, int &e, float &mant) {
  const int ex = (int)((f2u(d) >> 23) & 0xFF) - 127;  // d == 0 gives -127 -> -20, mant 0
  e = ex < -20 ? -20 : (ex > 0 ? 0 : ex);
  mant = __builtin_ldexpf(d, -e);
}

typedef uint32_t u4s __attribute__((ext_vector_type(4)));
#define PKV_LDS __attribute__((address_space(3)))

// ---- LDS staging of 32-key blocks. Rows (144 B = 9 slots of 16 B) of one KV head are
// placed at slot 9R + 4*(R/8): the 64 B gap after every 8 rows puts the four 8-row
// groups that a transposed V read touches at once on disjoint LDS banks.
constexpr int kSlots = 320;   // 5 loads of 64 lanes x 16 B; 304 slots used
constexpr int kStages = 3;
struct Stage {
  u4 k[kSlots];
  u4 v[kSlots];
};
__device__ __forceinline__ int row_slot(int R) { return 9 * R + 4 * (R >> 3); }

// Buffer resource of a byte range (raw, stride 0; out-of-range loads return zero).
__device__ __forceinline__ u4s make_rsrc(const void *base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  u4s r;
  r.x = __builtin_amdgcn_readfirstlane((uint32_t)p);
  r.y = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32) & 0xFFFFu);
  r.z = __builtin_amdgcn_readfirstlane(bytes);
  r.w = 0x00020000u;
  return r;
}

// One lane's part of staging a block: up to 5 16-byte pieces per tensor. Issued from
// inline asm so that the compiler's wait-count pass does not serialise the LDS reads
// behind these transfers; the kernel places its own s_waitcnt vmcnt before a stage is
// read.
struct LoadPlan {
  uint32_t voff[5];
  uint32_t valid;
};

__device__ __forceinline__ LoadPlan make_plan(int lane, uint32_t rs_t) {
  LoadPlan P;
  P.valid = 0;
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    const int slot = 64 * i + lane;
    const int G = slot / 76, w = slot % 76;
    const bool ok = G < 4 && w < 72;
    const int R = 8 * G + w / 9, piece = w % 9;
    P.voff[i] = ok ? (uint32_t)R * rs_t + 16u * (uint32_t)piece : 0u;
    P.valid |= (ok ? 1u : 0u) << i;
  }
  return P;
}

__device__ __forceinline__ void lds_dma16(uint32_t lds, uint32_t voff, u4s rsrc, uint32_t soff) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "buffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds), "v"(voff), "s"(rsrc), "s"(soff)
      : "memory");
}

__device__ __forceinline__ void issue_stage(Stage *st, const LoadPlan &P, u4s rk, u4s rv,
                                            uint32_t soff) {
  soff = __builtin_amdgcn_readfirstlane(soff);
  const uint32_t lk = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)((PKV_LDS void *)&st->k[0]));
  const uint32_t lv = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)((PKV_LDS void *)&st->v[0]));
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    if (P.valid & (1u << i)) {
      lds_dma16(lk + 1024u * i, P.voff[i], rk, soff);
      lds_dma16(lv + 1024u * i, P.voff[i], rv, soff);
    }
  }
}

// every lane issues exactly 10 loads per stage, so the count below is static
__device__ __forceinline__ void wait_stage_ready() {
  asm volatile("s_waitcnt vmcnt(20)" ::: "memory");  // the two younger stages may fly
}



struct WaveState {
  f4 acc[16];  // PV accumulators, tile T = 8h + 2*byte + hl
  f4 accm;     // min-term accumulator
  float m_run, lsum;
};

// ---- per-block phases. The loop runs P(i) and Q(i+1) in one branch-free region so
// the scheduler can overlap the MFMA chains, LDS reads and VALU work of two blocks.
struct QKOut {
  f4 s1[2], s2[2];  // per 16-key tile: sum_e (n*sc)_e q_e and sum_j m_j qsum_j
};

// Phase Q: K rows of a staged block -> raw QK sums; per-key d, dmin into the tables.
__device__ __forceinline__ void phase_q(const Stage &st, WaveTab &T, const h8 *qb, h4 q2,
                                        float sl2, const Masks &MK, int lane, QKOut &o) {
  const int r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int kk = 8 * (r >> 2) + 4 * t + (r & 3);
    const int sl = row_slot(kk);
    const u4 hd = st.k[sl];
    const u4 q0 = st.k[sl + 1 + 2 * g], q1 = st.k[sl + 2 + 2 * g];
    // lanes of one key (g = 0..3) store the same values
    T.kd[kk] = h2f(hd.x & 0xFFFF) * sl2;
    T.kdm[kk] = h2f(hd.x >> 16) * sl2;
    uint32_t sc0, sc1, mm;
    scale_min(hd.y, hd.z, hd.w, 2 * g, sc0, mm);
    scale_min(hd.y, hd.z, hd.w, 2 * g + 1, sc1, mm);
    const _Float16 f0 = (_Float16)(float)sc0, f1 = (_Float16)((float)sc1 * 0.0625f);
    const _Float16 c0 = (_Float16)(-1024.0f * (float)sc0), c1 = (_Float16)(-64.0f * (float)sc1);
    const h2 SC0 = {f0, f0}, SC1 = {f1, f1}, C0 = {c0, c0}, C1 = {c1, c1};
    const uint32_t qd[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    f4 s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint32_t d0 = qd[2 * s], d1 = qd[2 * s + 1];
      const uint32_t d0s = d0 >> 8, d1s = d1 >> 8;
      const uint32_t lw[4] = {and_or(d0, MK.lo, MK.magic), and_or(d0s, MK.lo, MK.magic),
                              and_or(d1, MK.lo, MK.magic), and_or(d1s, MK.lo, MK.magic)};
      const uint32_t hw[4] = {and_or(d0, MK.hi, MK.magic), and_or(d0s, MK.hi, MK.magic),
                              and_or(d1, MK.hi, MK.magic), and_or(d1s, MK.hi, MK.magic)};
      h8 lo, hi;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const h2 l2 = pk_fma(as_h2(lw[w]), SC0, C0);
        const h2 hh2 = pk_fma(as_h2(hw[w]), SC1, C1);
        lo[2 * w] = l2[0];
        lo[2 * w + 1] = l2[1];
        hi[2 * w] = hh2[0];
        hi[2 * w + 1] = hh2[1];
      }
      s1 = mfma32(lo, qb[s], s1);
      s1 = mfma32(hi, qb[4 + s], s1);
    }
    h4 a2;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      uint32_t scx, m;
      scale_min(hd.y, hd.z, hd.w, (4 * g + jj) & 7, scx, m);
      a2[jj] = g < 2 ? (_Float16)(float)m : (_Float16)0.0f;
    }
    o.s1[t] = s1;
    o.s2[t] = mfma16(a2, q2, f4{0.f, 0.f, 0.f, 0.f});
  }
}

// Cross-lane max through v_permlane{16,32}_swap: with both operands x, the two results
// hold x of lanes l and l ^ 16 (l ^ 32). The elements are copied to scalars before the
// bit cast: __builtin_bit_cast of a vector element r[1] reads element 0 (clang lowers
// it through the vector's address).
__device__ __forceinline__ float max_pair(uint32_t a, uint32_t b) {
  return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}
__device__ __forceinline__ float xmax16(float x) {  // max over lanes l and l ^ 16
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  return max_pair(r0, r1);
}
__device__ __forceinline__ float xmax32(float x) {  // max over lanes l and l ^ 32
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  return max_pair(r0, r1);
}

// Phase S: scores (log2 units) and the online softmax; p[k] for key 8g + k, head n % 8.
__device__ __forceinline__ void phase_s(const QKOut &o, WaveState &S, const WaveTab &T,
                                        int64_t key0, int64_t seq_k, int lane, float p[8]) {
  const int g = lane >> 4;
  float sc8[8];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kk = 8 * g + 4 * t + i;
      const float v1 = o.s1[t][i] + ror8(o.s1[t][i]);
      const float v2 = o.s2[t][i] + ror8(o.s2[t][i]);
      float sc = T.kd[kk] * v1 - T.kdm[kk] * v2;
      sc = fminf(fmaxf(sc, -kClampL2), kClampL2);
      sc8[4 * t + i] = key0 + kk < seq_k ? sc : -INFINITY;
    }
  float bm = sc8[0];
#pragma unroll
  for (int k = 1; k < 8; ++k) bm = fmaxf(bm, sc8[k]);
  bm = xmax32(xmax16(bm));
  if (__any(bm > S.m_run)) {
    const float m_new = fmaxf(S.m_run, bm);
    const float alpha = (S.m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(S.m_run - m_new);
    S.lsum *= alpha;
    S.m_run = m_new;
    float ai[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ai[i] = __shfl(alpha, 4 * (g & 1) + i);
#pragma unroll
    for (int T2 = 0; T2 < 16; ++T2)
#pragma unroll
      for (int i = 0; i < 4; ++i) S.acc[T2][i] *= ai[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) S.accm[i] *= ai[i];
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    p[k] = __builtin_amdgcn_exp2f(sc8[k] - S.m_run);
    S.lsum += p[k];
  }
}

// Phase P: V header tables, PV A/B operands and MFMAs, min term.
__device__ __forceinline__ void phase_p(const Stage &st, WaveState &S, WaveTab &T,
                                        const float p[8], const Masks &MK, int lane) {
  const int n = lane & 15, g = lane >> 4;
  // V header -> constant tables. Lane l handles key l % 32 and sub-blocks 4*(l/32)..+3.
  {
    const int kk = lane & 31, half = lane >> 5;
    const u4 vh = st.v[row_slot(kk)];
    int ed, em;
    float md, mm;
    split_scale(h2f(vh.x & 0xFFFF), ed, md);
    split_scale(h2f(vh.x >> 16), em, mm);
    (half ? T.vmdm : T.vmd)[kk] = half ? mm : md;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int j = 4 * half + jj;
      uint32_t sc, m;
      scale_min(vh.y, vh.z, vh.w, j, sc, m);
      const float scp = __builtin_ldexpf((float)sc, ed);
      T.vsc[j][kk] = (_Float16)((jj & 1) ? scp * 0.0625f : scp);
      T.vc[j][kk] = (_Float16)((jj & 1) ? -64.0f * scp : -1024.0f * scp);
      T.vm[j][kk] = (_Float16)__builtin_ldexpf((float)m, em);
    }
  }
  // V rows, transposed: dword at qs byte 64h + 4n of keys 8g..8g+7
  uint32_t vq[2][8];
  const uint32_t *v32 = reinterpret_cast<const uint32_t *>(st.v);
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int base = 4 * row_slot(8 * g + k) + 4 + n;
    vq[0][k] = v32[base];
    vq[1][k] = v32[base + 16];
  }
  // A: rows 0-7 p * mant(d), rows 8-15 p * mant(dmin)
  const float *mult = (n < 8) ? T.vmd : T.vmdm;
  h8 A;
#pragma unroll
  for (int k = 0; k < 8; ++k) A[k] = (_Float16)(p[k] * mult[8 * g + k]);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int c = 2 * h + (n >> 3);
    const h8 SL = *reinterpret_cast<const h8 *>(&T.vsc[2 * c][8 * g]);
    const h8 CL = *reinterpret_cast<const h8 *>(&T.vc[2 * c][8 * g]);
    const h8 SH = *reinterpret_cast<const h8 *>(&T.vsc[2 * c + 1][8 * g]);
    const h8 CH = *reinterpret_cast<const h8 *>(&T.vc[2 * c + 1][8 * g]);
#pragma unroll
    for (int byte = 0; byte < 4; ++byte) {
      const uint32_t sel = (uint32_t)byte | (0x0Cu << 8) | ((uint32_t)(4 + byte) << 16) | (0x0Cu << 24);
      h8 blo, bhi;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        const uint32_t x = __builtin_amdgcn_perm(vq[h][2 * pp + 1], vq[h][2 * pp], sel);
        const h2 lo = pk_fma(as_h2(and_or(x, MK.lo, MK.magic)),
                             h2{SL[2 * pp], SL[2 * pp + 1]}, h2{CL[2 * pp], CL[2 * pp + 1]});
        const h2 hi = pk_fma(as_h2(and_or(x, MK.hi, MK.magic)),
                             h2{SH[2 * pp], SH[2 * pp + 1]}, h2{CH[2 * pp], CH[2 * pp + 1]});
        blo[2 * pp] = lo[0];
        blo[2 * pp + 1] = lo[1];
        bhi[2 * pp] = hi[0];
        bhi[2 * pp + 1] = hi[1];
      }
      S.acc[8 * h + 2 * byte] = mfma32(A, blo, S.acc[8 * h + 2 * byte]);
      S.acc[8 * h + 2 * byte + 1] = mfma32(A, bhi, S.acc[8 * h + 2 * byte + 1]);
    }
  }
  // min term: C'[8 + head][j] += sum_k p * mant(dmin) * m_kj * 2^e_dmin
  const h8 Bm0 = *reinterpret_cast<const h8 *>(&T.vm[n & 7][8 * g]);
  const h8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
  S.accm = mfma32(A, n < 8 ? Bm0 : zero8, S.accm);
}

// e (0..255) of PV tile T at lane column n
__device__ __forceinline__ int tile_e(int T, int n) {
  const int h = T >> 3, byte = (T >> 1) & 3, hl = T & 1;
  const int c = 2 * h + (n >> 3);
  return 64 * c + 32 * hl + 4 * (n & 7) + byte;
}

__global__ __launch_bounds__(kThreads) void q4k_decode_kernel(DecodeArgs a) {
  __shared__ Smem sm;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kv = wave >> 1, wsub = wave & 1;
  const int b = blockIdx.y, wg = blockIdx.x;
  const int n = lane & 15, g = lane >> 4;

  // ---- fused append: workgroups past the main ones each quantize one new row and
  // publish it dequantized for the combine step (which attends to the new key)
  if (wg >= a.nwg_main) {
    const int rowid = wg - a.nwg_main;  // 0: K kv0, 1: K kv1, 2: V kv0, 3: V kv1
    const int p = rowid >> 1, kvr = rowid & 1;
    const float *src = (p ? a.v_new : a.k_new) + ((int64_t)b * 2 + kvr) * 256;
    uint8_t *dst = (p ? a.vw : a.kw) + b * a.rs_b + a.t_new * a.rs_t + kvr * a.rs_h;
    float deq;
    q4k_quantize_superblock_lanes(src[tid], dst, &sm.quant, tid, &deq);
    a.dq[((int64_t)b * 4 + rowid) * 256 + tid] = deq;
    return;
  }

  // ---- q operands (fp16 hi/lo, columns 0-7 hi, 8-15 lo) into LDS. q is staged in the
  // (not yet used) table area with coalesced loads first.
  {
    float *qf = &sm.qsetup.qf[0][0];
    float *qs = &sm.qsetup.qs[0][0];
    const float4 *src4 = reinterpret_cast<const float4 *>(a.q + (int64_t)b * 16 * 256);
    for (int x = tid; x < 16 * 256 / 4; x += kThreads) reinterpret_cast<float4 *>(qf)[x] = src4[x];
    __syncthreads();
    if (tid < 128) {
      const float *qq = qf + (tid >> 3) * 256 + 32 * (tid & 7);
      float sacc = 0.0f;
#pragma unroll
      for (int e = 0; e < 32; ++e) sacc += qq[e];
      qs[tid] = sacc;
    }
    __syncthreads();
    constexpr int perm[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    for (int x = tid; x < 2 * 8 * 64; x += kThreads) {
      const int ln = x & 63, st = (x >> 6) & 7, kvx = x >> 9;
      const int nn = ln & 15, gg = ln >> 4;
      const float *qrow = qf + (8 * kvx + (nn & 7)) * 256 + 64 * gg + 32 * (st >> 2) + 8 * (st & 3);
      h8 val;
#pragma unroll
      for (int slot = 0; slot < 8; ++slot) {
        const float qv = qrow[perm[slot]];
        const _Float16 hi = (_Float16)qv;
        val[slot] = (nn < 8) ? hi : (_Float16)(qv - (float)hi);
      }
      sm.qsetup.qb[kvx][st][ln] = val;
    }
    if (tid < 128) {
      const int ln = tid & 63, kvx = tid >> 6;
      const int nn = ln & 15, gg = ln >> 4;
      h4 val = {0, 0, 0, 0};
      if (gg < 2) {
#pragma unroll
        for (int slot = 0; slot < 4; ++slot) {
          const float sv = qs[(8 * kvx + (nn & 7)) * 8 + 4 * gg + slot];
          const _Float16 hi = (_Float16)sv;
          val[slot] = (nn < 8) ? hi : (_Float16)(sv - (float)hi);
        }
      }
      sm.qsetup.q2[kvx][ln] = val;
    }
  }
  __syncthreads();
  h8 qb[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) qb[s] = sm.qsetup.qb[kv][s][lane];
  const h4 q2 = sm.qsetup.q2[kv][lane];
  __syncthreads();  // the staging area becomes the wave tables

  // ---- block range of this workgroup
  const int b0 = wg * a.bpw;
  const int b1 = b0 + a.bpw < a.nblk ? b0 + a.bpw : a.nblk;
  WaveState S;
#pragma unroll
  for (int T2 = 0; T2 < 16; ++T2) S.acc[T2] = f4{0.f, 0.f, 0.f, 0.f};
  S.accm = f4{0.f, 0.f, 0.f, 0.f};
  S.m_run = -INFINITY;
  S.lsum = 0.0f;
  WaveTab &T = sm.run.tab[wave];
  const int kvu = __builtin_amdgcn_readfirstlane(kv);
  const uint8_t *kbase = a.k + b * a.rs_b + kvu * a.rs_h;
  const uint8_t *vbase = a.v + b * a.rs_b + kvu * a.rs_h;
  const uint32_t rs_t = (uint32_t)a.rs_t;
  // rows of keys [0, seq_k) of this head; loads past them return zeros (and are masked)
  const uint32_t span = (uint32_t)(a.seq_k - 1) * rs_t + 144u;
  const u4s rk = make_rsrc(kbase, span), rv = make_rsrc(vbase, span);
  const LoadPlan P = make_plan(lane, rs_t);
  const Masks MK = {vconst(0x000F000Fu), vconst(0x00F000F0u), vconst(0x64006400u)};
  Stage *stages = reinterpret_cast<Stage *>(sm.run.stages) + wave * kStages;
  // Three-stage pipeline: blocks first, first+2, first+4, ... of this wave are staged
  // into LDS two ahead of the one being processed. Every iteration issues one stage
  // (a block past the end reads out of range, which moves no data) so the wait count
  // stays constant.
  const int first = b0 + wsub;
  const int nmine = first < b1 ? (b1 - first + 1) / 2 : 0;
  auto soff_of = [&](int i) -> uint32_t {
    return i < nmine ? (uint32_t)(first + 2 * i) * kBlk * rs_t : 0xFFFFFF00u;
  };
  if (nmine > 0) {
    issue_stage(&stages[0], P, rk, rv, soff_of(0));
    issue_stage(&stages[1], P, rk, rv, soff_of(1));
    issue_stage(&stages[2], P, rk, rv, soff_of(2));
    asm volatile("s_waitcnt vmcnt(20)" ::: "memory");  // stage 0 landed
    QKOut qo;
    float pv[8];
    phase_q(stages[0], T, qb, q2, a.sl2, MK, lane, qo);
    phase_s(qo, S, T, (int64_t)first * kBlk, a.seq_k, lane, pv);
    for (int i = 0; i < nmine; ++i) {
      asm volatile("s_waitcnt vmcnt(10)" ::: "memory");  // stage i+1 landed
      // P(i) and Q(i+1) form one straight-line region
      phase_p(stages[i % kStages], S, T, pv, MK, lane);
      phase_q(stages[(i + 1) % kStages], T, qb, q2, a.sl2, MK, lane, qo);
      // stage i is refilled with block i+3 once its LDS reads have completed
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      issue_stage(&stages[i % kStages], P, rk, rv, soff_of(i + 3));
      if (i + 1 < nmine) phase_s(qo, S, T, (int64_t)(first + 2 * (i + 1)) * kBlk, a.seq_k, lane, pv);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  // ---- per-wave reductions
  S.lsum += __shfl_xor(S.lsum, 16);
  S.lsum += __shfl_xor(S.lsum, 32);
  __syncthreads();  // all waves done with sm.run before it is reused for merging
  // min-term table per wave: accm rows 8 + 4(g-2) + i = head 4(g-2)+i, column j = n
  if (g >= 2 && n < 8) {
#pragma unroll
    for (int i = 0; i < 4; ++i) sm.merge.cmin[wave][4 * (g - 2) + i][n] = S.accm[i];
  }
  __syncthreads();
  // O'[head][e] = acc - cmin[head][e / 32] (lanes g < 2 hold rows 4g+i = head 4g+i)
  float o[16][4];
#pragma unroll
  for (int T2 = 0; T2 < 16; ++T2) {
    const int e = tile_e(T2, n);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[T2][i] = S.acc[T2][i] - sm.merge.cmin[wave][(4 * g + i) & 7][e >> 5];
  }
  // ---- merge the two waves of each KV head through LDS
  float mw = S.m_run;  // for head n % 8
  float lw = S.lsum;
  __syncthreads();
  if (wsub == 1) {
    if (g < 2) {
#pragma unroll
      for (int T2 = 0; T2 < 16; ++T2)
#pragma unroll
        for (int i = 0; i < 4; ++i) sm.merge.o[kv][4 * g + i][tile_e(T2, n)] = o[T2][i];
    }
    if (g == 0 && n < 8) {
      sm.merge.m[kv][n] = mw;
      sm.merge.l[kv][n] = lw;
    }
  }
  __syncthreads();
  if (wsub == 0) {
    const float mo = sm.merge.m[kv][n & 7], lo2 = sm.merge.l[kv][n & 7];
    const float M = fmaxf(mw, mo);
    const float fa = (mw == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
    const float fb = (mo == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mo - M);
    float fai[4], fbi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // o rows are head 4g+i: factors of heads 4(g&1)+i
      fai[i] = __shfl(fa, 4 * (g & 1) + i);
      fbi[i] = __shfl(fb, 4 * (g & 1) + i);
    }
    lw = lw * fa + lo2 * fb;
    mw = M;
    float *dst = a.part + ((int64_t)b * a.nwg_main + wg) * 16 * 258;
    if (g < 2) {
#pragma unroll
      for (int T2 = 0; T2 < 16; ++T2) {
        const int e = tile_e(T2, n);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          dst[(8 * kv + 4 * g + i) * 258 + e] =
              o[T2][i] * fai[i] + sm.merge.o[kv][4 * g + i][e] * fbi[i];
      }
    }
    if (g == 0 && n < 8) {
      dst[(8 * kv + n) * 258 + 256] = mw;
      dst[(8 * kv + n) * 258 + 257] = lw;
    }
  }
}

// out[b][h][e] = sum_w o_w 2^(m_w - M) / sum_w l_w 2^(m_w - M).
// One workgroup per (head, 64-wide slice of e, batch); 4 thread groups split the partials.
constexpr int kMaxPartials = 1024;
// out[b][h][e] = (sum_w o_w 2^(m_w - M) + [new key]) / (sum_w l_w 2^(m_w - M) + [new key]).
// One workgroup per (head, 64-wide slice of e, batch); 4 thread groups split the
// partials. For a fused decode step the appended key enters here, from its exactly
// dequantized K and V rows: score = clamp(q . k_new * scale), weight 2^(score - M).
__global__ __launch_bounds__(256) void q4k_decode_combine_kernel(const float *part, int nwg,
                                                                 const float *q, const float *dq,
                                                                 float sl2, float *out) {
  __shared__ float wts[kMaxPartials];
  __shared__ float red[256];
  __shared__ float acc4[4][64];
  const int h = blockIdx.x >> 2, e0 = 64 * (blockIdx.x & 3), b = blockIdx.y;
  const int tid = threadIdx.x;
  const float *P = part + (int64_t)b * nwg * 16 * 258 + h * 258;
  // new key's score (log2 units), every thread gets it
  float s_new = -INFINITY;
  if (dq != nullptr) {
    red[tid] = q[((int64_t)b * 16 + h) * 256 + tid] * dq[((int64_t)b * 4 + (h >> 3)) * 256 + tid];
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
      if (tid < o) red[tid] += red[tid + o];
      __syncthreads();
    }
    s_new = fminf(fmaxf(red[0] * sl2, -kClampL2), kClampL2);
    __syncthreads();
  }
  float M = s_new;
  for (int w = tid; w < nwg; w += 256) M = fmaxf(M, P[(int64_t)w * 16 * 258 + 256]);
  red[tid] = M;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (tid < o) red[tid] = fmaxf(red[tid], red[tid + o]);
    __syncthreads();
  }
  M = red[0];
  __syncthreads();
  float L = 0.0f;
  for (int w = tid; w < nwg; w += 256) {
    const float mw = P[(int64_t)w * 16 * 258 + 256];
    const float f = (mw == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
    wts[w] = f;
    L += f * P[(int64_t)w * 16 * 258 + 257];
  }
  red[tid] = L;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (tid < o) red[tid] += red[tid + o];
    __syncthreads();
  }
  const float f_new = (s_new == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(s_new - M);
  L = red[0] + f_new;
  const int e = tid & 63, r = tid >> 6;
  float acc = 0.0f;
#pragma unroll 8
  for (int w = r; w < nwg; w += 4) acc += wts[w] * P[(int64_t)w * 16 * 258 + e0 + e];
  acc4[r][e] = acc;
  __syncthreads();
  if (tid < 64) {
    float sum = acc4[0][tid] + acc4[1][tid] + acc4[2][tid] + acc4[3][tid];
    if (dq != nullptr) sum += f_new * dq[((int64_t)b * 4 + 2 + (h >> 3)) * 256 + e0 + tid];
    out[((int64_t)b * 16 + h) * 256 + e0 + tid] = L > 0.0f ? sum / L : 0.0f;
  }
}

}  // namespace

int launch_attend_mfma(const AttnArgs &a, const float *k_new, const float *v_new, uint8_t *kc,
                       uint8_t *vc, int64_t t_new, Workspace &ws, hipStream_t s) {
  if (a.quant != PKV_QUANT_Q4K || a.head_dim != 256 || a.num_heads != 16 ||
      a.num_kv_heads != 2 || a.l != 1)
    return PKV_ERR_UNSUPPORTED;
  // decode only: the single query sees every key
  if (a.causal && a.q_offset + 1 < a.seq_k) return PKV_ERR_UNSUPPORTED;
  const bool fused = k_new != nullptr;
  // rows are addressed with 32-bit offsets (key * row stride) from a per-head base
  if (a.rs.t >= (1 << 24) || a.seq_k >= (1 << 24) ||
      (uint64_t)a.seq_k * (uint64_t)a.rs.t >= (1ull << 32))
    return PKV_ERR_UNSUPPORTED;
  DecodeArgs d;
  d.q = a.q;
  d.k = a.k;
  d.v = a.v;
  d.kw = kc;
  d.vw = vc;
  d.rs_b = a.rs.b;
  d.rs_t = a.rs.t;
  d.rs_h = a.rs.h;
  d.seq_k = fused ? a.seq_k - 1 : a.seq_k;  // old keys; the new one joins in the combine
  d.nblk = (int)((d.seq_k + kBlk - 1) / kBlk);
  int nwg = (d.nblk + 1) / 2;
  if (nwg > kMainWGs) nwg = kMainWGs;  // nwg <= kMaxPartials
  if (nwg < 1) nwg = 1;
  d.bpw = (d.nblk + nwg - 1) / nwg;
  d.bpw = (d.bpw + 1) / 2 * 2;
  if (d.bpw < 2) d.bpw = 2;
  nwg = (d.nblk + d.bpw - 1) / d.bpw;
  if (nwg < 1) nwg = 1;
  d.nwg_main = nwg;
  d.sl2 = a.scale * kLog2e;
  d.k_new = k_new;
  d.v_new = v_new;
  d.t_new = t_new;
  const size_t part_floats = (size_t)a.batch * nwg * 16 * 258;
  const size_t need = (part_floats + (size_t)a.batch * 4 * 256) * sizeof(float);
  int rc = ws.reserve(need);
  if (rc) return rc;
  d.part = static_cast<float *>(ws.ptr);
  d.dq = d.part + part_floats;
  hipLaunchKernelGGL(q4k_decode_kernel, dim3((unsigned)(nwg + (fused ? 4 : 0)), (unsigned)a.batch),
                     dim3(kThreads), 0, s, d);
  PKV_HIP(hipGetLastError());
  hipLaunchKernelGGL(q4k_decode_combine_kernel, dim3(64, (unsigned)a.batch), dim3(256), 0, s,
                     d.part, nwg, a.q, fused ? d.dq : nullptr, d.sl2, a.out);
  PKV_HIP(hipGetLastError());
  return PKV_OK;
}

}  // namespace pkv
