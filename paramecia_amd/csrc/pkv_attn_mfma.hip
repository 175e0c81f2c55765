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

constexpr int kThreads = 512;
constexpr int kBlk = 32;
constexpr int kMainWGs = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kClampL2 = 100.0f * 1.4426950408889634f;  // +-100 nats in log2 units

struct DecodeArgs {
  const float *q;  // [B][16][256]
  const uint8_t *k, *v;
  uint8_t *kw, *vw;
  int64_t rs_b, rs_t, rs_h;
  int64_t seq_k;
  int nblk, nwg_main, bpw;
  float sl2;  // scale * log2(e)
  const float *k_new, *v_new;  // [B][2][256] or null
  int64_t t_new;
  float *part;  // [B][nwg_main + 1][16][258]
};

// Per-wave tables rebuilt for every 32-key block.
struct WaveTab {
  float kd[kBlk], kdm[kBlk];                     // K: d*sl2, dmin*sl2
  float vmd[kBlk], vmdm[kBlk];                   // V: mantissas of d and dmin
  _Float16 vsc[8][kBlk], vc[8][kBlk], vm[8][kBlk];  // V: fp16 constants [j][key]
};

struct Smem {
  union {
    struct {
      h8 qb[2][8][64];  // QK B operands [kv][step][lane]
      h4 q2[2][64];     // S2 B operands [kv][lane]
      WaveTab tab[8];
    } run;
    struct {
      float o[4][8][256];  // merge staging for up to 4 waves
      float m[4][8], l[4][8];
      float cmin[8][8][8];  // per wave [head][j]
    } merge;
    Q4kScratch quant[2];
  };
};

__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t o) {
  return (x & m) | o;
}
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
  const int jj = j & 3;
  const uint32_t b_lo = (s0 >> (8 * jj)) & 0xFF;  // byte j (j < 4) or j-4
  const uint32_t b_mid = (s1 >> (8 * jj)) & 0xFF; // byte j+4 (j < 4) or j
  const uint32_t b_hi = (s2 >> (8 * jj)) & 0xFF;  // byte j+4 (j >= 4)
  if (j < 4) {
    sc = b_lo & 63;
    m = b_mid & 63;
  } else {
    sc = (b_hi & 0xF) | ((b_lo >> 6) << 4);
    m = (b_hi >> 4) | ((b_mid >> 6) << 4);
  }
}

// exponent e in [-20, 0] and mantissa d * 2^-e of a non-negative f16 scale
__device__ __forceinline__ void split_scale(float d, int &e, float &mant) {
  if (d == 0.0f) {
    e = -20;
    mant = 0.0f;
    return;
  }
  int ex = (int)((f2u(d) >> 23) & 0xFF) - 127;
  e = ex < -20 ? -20 : (ex > 0 ? 0 : ex);
  mant = __builtin_ldexpf(d, -e);
}

struct BlockLoads {
  u4 khdr[2], kq0[2], kq1[2];  // per QK tile
  uint32_t vq[2][8];           // [dword set][key]
  u4 vhdr;
};

__device__ __forceinline__ const uint8_t *row_ptr(const uint8_t *base, const DecodeArgs &a,
                                                  int b, int64_t key, int kv) {
  return base + b * a.rs_b + key * a.rs_t + kv * a.rs_h;
}

__device__ __forceinline__ void load_block(BlockLoads &L, const DecodeArgs &a, int b, int kv,
                                           int bi, int lane) {
  const int r = lane & 15, g = lane >> 4;
  const int64_t kb = (int64_t)bi * kBlk, last = a.seq_k - 1;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    int64_t key = kb + 8 * (r >> 2) + 4 * t + (r & 3);
    key = key > last ? last : key;
    const uint8_t *row = row_ptr(a.k, a, b, key, kv);
    L.khdr[t] = *reinterpret_cast<const u4 *>(row);
    L.kq0[t] = *reinterpret_cast<const u4 *>(row + 16 + 32 * g);
    L.kq1[t] = *reinterpret_cast<const u4 *>(row + 32 + 32 * g);
  }
  const int n = lane & 15;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    int64_t key = kb + 8 * g + k;
    key = key > last ? last : key;
    const uint8_t *row = row_ptr(a.v, a, b, key, kv);
    L.vq[0][k] = *reinterpret_cast<const uint32_t *>(row + 16 + 4 * n);
    L.vq[1][k] = *reinterpret_cast<const uint32_t *>(row + 80 + 4 * n);
  }
  int64_t key = kb + (lane & 31);
  key = key > last ? last : key;
  L.vhdr = *reinterpret_cast<const u4 *>(row_ptr(a.v, a, b, key, kv));
}

struct WaveState {
  f4 acc[16];  // PV accumulators, tile T = 8h + 2*byte + hl
  f4 accm;     // min-term accumulator
  float m_run, lsum;
};

__device__ __forceinline__ void process_block(const BlockLoads &L, WaveState &S, WaveTab &T,
                                              const h8 *qb, h4 q2, const DecodeArgs &a, int bi,
                                              int lane) {
  const int n = lane & 15, g = lane >> 4;
  // ---- V header -> constant tables (lanes 0-31: scale tables, 32-63: min tables)
  {
    const int kk = lane & 31;
    const uint32_t s0 = L.vhdr.y, s1 = L.vhdr.z, s2 = L.vhdr.w;
    const float d = f16_to_f32((uint16_t)(L.vhdr.x & 0xFFFF));
    const float dmin = f16_to_f32((uint16_t)(L.vhdr.x >> 16));
    if (lane < 32) {
      int e;
      float mant;
      split_scale(d, e, mant);
      T.vmd[kk] = mant;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint32_t sc, m;
        scale_min(s0, s1, s2, j, sc, m);
        const float scp = __builtin_ldexpf((float)sc, e);
        T.vsc[j][kk] = (_Float16)((j & 1) ? scp * 0.0625f : scp);
        T.vc[j][kk] = (_Float16)((j & 1) ? -64.0f * scp : -1024.0f * scp);
      }
    } else {
      int e;
      float mant;
      split_scale(dmin, e, mant);
      T.vmdm[kk] = mant;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint32_t sc, m;
        scale_min(s0, s1, s2, j, sc, m);
        T.vm[j][kk] = (_Float16)__builtin_ldexpf((float)m, e);
      }
    }
  }
  // ---- QK for the two 16-key tiles
  float sc8[8];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const u4 hd = L.khdr[t];
    const float d = f16_to_f32((uint16_t)(hd.x & 0xFFFF));
    const float dmin = f16_to_f32((uint16_t)(hd.x >> 16));
    const int r = lane & 15;
    const int kk = 8 * (r >> 2) + 4 * t + (r & 3);
    if (g == 0) {
      T.kd[kk] = d * a.sl2;
      T.kdm[kk] = dmin * a.sl2;
    }
    uint32_t sc0, sc1, mm;
    scale_min(hd.y, hd.z, hd.w, 2 * g, sc0, mm);
    scale_min(hd.y, hd.z, hd.w, 2 * g + 1, sc1, mm);
    const _Float16 f0 = (_Float16)(float)sc0, f1 = (_Float16)((float)sc1 * 0.0625f);
    const h2 SC0 = {f0, f0}, SC1 = {f1, f1};
    const _Float16 c0 = (_Float16)(-1024.0f * (float)sc0), c1 = (_Float16)(-64.0f * (float)sc1);
    const h2 C0 = {c0, c0}, C1 = {c1, c1};
    f4 s1 = {0.f, 0.f, 0.f, 0.f};
    const uint32_t qd[8] = {L.kq0[t].x, L.kq0[t].y, L.kq0[t].z, L.kq0[t].w,
                            L.kq1[t].x, L.kq1[t].y, L.kq1[t].z, L.kq1[t].w};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint32_t d0 = qd[2 * s], d1 = qd[2 * s + 1];
      const uint32_t d0s = d0 >> 8, d1s = d1 >> 8;
      h8 lo, hi;
      const uint32_t lw[4] = {and_or(d0, 0x000F000Fu, 0x64006400u), and_or(d0s, 0x000F000Fu, 0x64006400u),
                              and_or(d1, 0x000F000Fu, 0x64006400u), and_or(d1s, 0x000F000Fu, 0x64006400u)};
      const uint32_t hw[4] = {and_or(d0, 0x00F000F0u, 0x64006400u), and_or(d0s, 0x00F000F0u, 0x64006400u),
                              and_or(d1, 0x00F000F0u, 0x64006400u), and_or(d1s, 0x00F000F0u, 0x64006400u)};
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
    // S2 = sum_j m_j * qsum_j
    h4 a2 = {0, 0, 0, 0};
    if (g < 2) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        uint32_t scx, m;
        scale_min(hd.y, hd.z, hd.w, 4 * g + jj, scx, m);
        a2[jj] = (_Float16)(float)m;
      }
    }
    f4 s2 = {0.f, 0.f, 0.f, 0.f};
    s2 = mfma16(a2, q2, s2);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key_local = 8 * g + 4 * t + i;
      const float v1 = s1[i] + ror8(s1[i]);
      const float v2 = s2[i] + ror8(s2[i]);
      float sc = T.kd[key_local] * v1 - T.kdm[key_local] * v2;
      sc = fminf(fmaxf(sc, -kClampL2), kClampL2);
      if ((int64_t)bi * kBlk + key_local >= a.seq_k) sc = -INFINITY;
      sc8[4 * t + i] = sc;
    }
  }
  // ---- online softmax (head n % 8; lanes n and n+8 hold the same values)
  float bm = sc8[0];
#pragma unroll
  for (int k = 1; k < 8; ++k) bm = fmaxf(bm, sc8[k]);
  bm = fmaxf(bm, __shfl_xor(bm, 16));
  bm = fmaxf(bm, __shfl_xor(bm, 32));
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
  float p[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    p[k] = __builtin_amdgcn_exp2f(sc8[k] - S.m_run);
    S.lsum += p[k];
  }
  // ---- PV A operand: rows 0-7 p * mant(d), rows 8-15 p * mant(dmin)
  const float *mult = (n < 8) ? T.vmd : T.vmdm;
  h8 A;
#pragma unroll
  for (int k = 0; k < 8; ++k) A[k] = (_Float16)(p[k] * mult[8 * g + k]);
  // ---- PV B operands and MFMAs
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
        const uint32_t x = __builtin_amdgcn_perm(L.vq[h][2 * pp + 1], L.vq[h][2 * pp], sel);
        const h2 lo = pk_fma(as_h2(and_or(x, 0x000F000Fu, 0x64006400u)),
                             h2{SL[2 * pp], SL[2 * pp + 1]}, h2{CL[2 * pp], CL[2 * pp + 1]});
        const h2 hi = pk_fma(as_h2(and_or(x, 0x00F000F0u, 0x64006400u)),
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
  // ---- min term: C'[8 + head][j] += sum_k p * mant(dmin) * m_kj * 2^e_dmin
  h8 Bm = {0, 0, 0, 0, 0, 0, 0, 0};
  if (n < 8) Bm = *reinterpret_cast<const h8 *>(&T.vm[n][8 * g]);
  S.accm = mfma32(A, Bm, S.accm);
  __builtin_amdgcn_wave_barrier();
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
  const int kv = wave >> 2, wsub = wave & 3;
  const int b = blockIdx.y, wg = blockIdx.x;
  const bool tail = wg == a.nwg_main;
  const int n = lane & 15, g = lane >> 4;

  // ---- fused append: the tail workgroup quantizes the new token's 4 rows first
  if (tail && a.k_new != nullptr) {
    const int half = tid >> 8, t2 = tid & 255;
#pragma unroll 1
    for (int round = 0; round < 2; ++round) {
      const int rowid = 2 * round + half;  // 0: K kv0, 1: K kv1, 2: V kv0, 3: V kv1
      const int p = rowid >> 1, kvr = rowid & 1;
      const float *src = (p ? a.v_new : a.k_new) + ((int64_t)b * 2 + kvr) * 256;
      uint8_t *dst = (p ? a.vw : a.kw) + b * a.rs_b + a.t_new * a.rs_t + kvr * a.rs_h;
      q4k_quantize_superblock_lanes(src[t2], dst, &sm.quant[half], t2);
    }
    __threadfence_block();
    __syncthreads();
  }

  // ---- q operands (fp16 hi/lo, columns 0-7 hi, 8-15 lo) into LDS
  const float *qb_src = a.q + (int64_t)b * 16 * 256;
  for (int x = tid; x < 2 * 8 * 64 * 8; x += kThreads) {
    const int slot = x & 7, ln = (x >> 3) & 63, s = (x >> 9) & 7, kvx = x >> 12;
    const int nn = ln & 15, gg = ln >> 4;
    const int perm[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    const int e = 64 * gg + 32 * (s >> 2) + 8 * (s & 3) + perm[slot];
    const float qv = qb_src[(8 * kvx + (nn & 7)) * 256 + e];
    const _Float16 hi = (_Float16)qv;
    const _Float16 lo = (_Float16)(qv - (float)hi);
    sm.run.qb[kvx][s][ln][slot] = (nn < 8) ? hi : lo;
  }
  for (int x = tid; x < 2 * 64 * 4; x += kThreads) {
    const int slot = x & 3, ln = (x >> 2) & 63, kvx = x >> 8;
    const int nn = ln & 15, gg = ln >> 4;
    _Float16 val = 0;
    if (gg < 2) {
      const int j = 4 * gg + slot;
      const float *qq = qb_src + (8 * kvx + (nn & 7)) * 256 + 32 * j;
      float s = 0.0f;
      for (int e = 0; e < 32; ++e) s += qq[e];
      const _Float16 hi = (_Float16)s;
      val = (nn < 8) ? hi : (_Float16)(s - (float)hi);
    }
    sm.run.q2[kvx][ln][slot] = val;
  }
  __syncthreads();
  h8 qb[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) qb[s] = sm.run.qb[kv][s][lane];
  const h4 q2 = sm.run.q2[kv][lane];

  // ---- block range
  int b0, b1;
  if (tail) {
    b0 = a.nblk - 1;
    b1 = a.nblk;
  } else {
    b0 = wg * a.bpw;
    b1 = b0 + a.bpw;
    if (b1 > a.nblk - 1) b1 = a.nblk - 1;
  }
  WaveState S;
#pragma unroll
  for (int T2 = 0; T2 < 16; ++T2) S.acc[T2] = f4{0.f, 0.f, 0.f, 0.f};
  S.accm = f4{0.f, 0.f, 0.f, 0.f};
  S.m_run = -INFINITY;
  S.lsum = 0.0f;
  WaveTab &T = sm.run.tab[wave];
  int bi = b0 + wsub;
  if (bi < b1) {
    BlockLoads cur;
    load_block(cur, a, b, kv, bi, lane);
    for (; bi < b1; bi += 4) {
      BlockLoads nxt;
      const bool more = bi + 4 < b1;
      if (more) load_block(nxt, a, b, kv, bi + 4, lane);
      process_block(cur, S, T, qb, q2, a, bi, lane);
      if (more) cur = nxt;
    }
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
  // ---- merge the 4 waves of each KV head (pairwise through LDS)
  float mw = S.m_run;  // for head n % 8
  float lw = S.lsum;
#pragma unroll 1
  for (int step = 2; step >= 1; step >>= 1) {
    __syncthreads();
    const bool writer = wsub >= step && wsub < 2 * step;
    const int slot = kv * 2 + (wsub - step);  // staging slot (0..3)
    if (writer) {
      if (g < 2) {
#pragma unroll
        for (int T2 = 0; T2 < 16; ++T2)
#pragma unroll
          for (int i = 0; i < 4; ++i) sm.merge.o[slot][4 * g + i][tile_e(T2, n)] = o[T2][i];
      }
      if (g == 0 && n < 8) {
        sm.merge.m[slot][n] = mw;
        sm.merge.l[slot][n] = lw;
      }
    }
    __syncthreads();
    if (wsub < step) {
      const int src = kv * 2 + wsub;
      const float mo = sm.merge.m[src][n & 7], lo2 = sm.merge.l[src][n & 7];
      const float M = fmaxf(mw, mo);
      const float fa = (mw == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
      const float fb = (mo == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mo - M);
      // o rows are head 4g+i: need factors of heads 4(g&1)+i
      float fai[4], fbi[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        fai[i] = __shfl(fa, 4 * (g & 1) + i);
        fbi[i] = __shfl(fb, 4 * (g & 1) + i);
      }
      if (g < 2) {
#pragma unroll
        for (int T2 = 0; T2 < 16; ++T2)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            o[T2][i] = o[T2][i] * fai[i] + sm.merge.o[src][4 * g + i][tile_e(T2, n)] * fbi[i];
      }
      lw = lw * fa + lo2 * fb;
      mw = M;
    }
  }
  // ---- write the workgroup partial: [16 heads][256 e | m | l]
  if (wsub == 0) {
    float *dst = a.part + ((int64_t)b * (a.nwg_main + 1) + wg) * 16 * 258;
    if (g < 2) {
#pragma unroll
      for (int T2 = 0; T2 < 16; ++T2)
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[(8 * kv + 4 * g + i) * 258 + tile_e(T2, n)] = o[T2][i];
    }
    if (g == 0 && n < 8) {
      dst[(8 * kv + n) * 258 + 256] = mw;
      dst[(8 * kv + n) * 258 + 257] = lw;
    }
  }
}

// out[b][h][e] = sum_w o_w e^(m_w - M) / sum_w l_w e^(m_w - M); one workgroup per (b, h).
__global__ __launch_bounds__(256) void q4k_decode_combine_kernel(const float *part, int nwg,
                                                                 float *out) {
  const int h = blockIdx.x, b = blockIdx.y, e = threadIdx.x;
  const float *P = part + (int64_t)b * nwg * 16 * 258 + h * 258;
  float M = -INFINITY;
  for (int w = 0; w < nwg; ++w) M = fmaxf(M, P[(int64_t)w * 16 * 258 + 256]);
  float acc = 0.0f, L = 0.0f;
  for (int w = 0; w < nwg; ++w) {
    const float mw = P[(int64_t)w * 16 * 258 + 256];
    const float f = (mw == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
    acc += f * P[(int64_t)w * 16 * 258 + e];
    L += f * P[(int64_t)w * 16 * 258 + 257];
  }
  out[((int64_t)b * 16 + h) * 256 + e] = L > 0.0f ? acc / L : 0.0f;
}

}  // namespace

int launch_attend_mfma(const AttnArgs &a, const float *k_new, const float *v_new, uint8_t *kc,
                       uint8_t *vc, int64_t t_new, Workspace &ws, hipStream_t s) {
  if (a.quant != PKV_QUANT_Q4K || a.head_dim != 256 || a.num_heads != 16 ||
      a.num_kv_heads != 2 || a.l != 1)
    return PKV_ERR_UNSUPPORTED;
  // decode only: the single query sees every key
  if (a.causal && a.q_offset + 1 < a.seq_k) return PKV_ERR_UNSUPPORTED;
  DecodeArgs d;
  d.q = a.q;
  d.k = a.k;
  d.v = a.v;
  d.kw = kc;
  d.vw = vc;
  d.rs_b = a.rs.b;
  d.rs_t = a.rs.t;
  d.rs_h = a.rs.h;
  d.seq_k = a.seq_k;
  d.nblk = (int)((a.seq_k + kBlk - 1) / kBlk);
  const int main_blocks = d.nblk - 1;
  int nwg = (main_blocks + 3) / 4;
  if (nwg > kMainWGs) nwg = kMainWGs;
  if (nwg < 1) nwg = 1;
  d.bpw = (main_blocks + nwg - 1) / nwg;
  d.bpw = (d.bpw + 3) / 4 * 4;
  if (d.bpw < 4) d.bpw = 4;
  nwg = (main_blocks + d.bpw - 1) / d.bpw;
  if (nwg < 1) nwg = 1;
  d.nwg_main = nwg;
  d.sl2 = a.scale * kLog2e;
  d.k_new = k_new;
  d.v_new = v_new;
  d.t_new = t_new;
  const size_t need = (size_t)a.batch * (nwg + 1) * 16 * 258 * sizeof(float);
  int rc = ws.reserve(need);
  if (rc) return rc;
  d.part = static_cast<float *>(ws.ptr);
  hipLaunchKernelGGL(q4k_decode_kernel, dim3((unsigned)(nwg + 1), (unsigned)a.batch),
                     dim3(kThreads), 0, s, d);
  PKV_HIP(hipGetLastError());
  hipLaunchKernelGGL(q4k_decode_combine_kernel, dim3(16, (unsigned)a.batch), dim3(256), 0, s,
                     d.part, nwg + 1, a.out);
  PKV_HIP(hipGetLastError());
  return PKV_OK;
}

}  // namespace pkv
