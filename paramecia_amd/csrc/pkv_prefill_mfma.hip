// MFMA prefill-chunk attention over a Q4K cache for the Qwen3-Next full-attention shape
// (16 query heads, 2 KV heads, head_dim 256), gfx950.
//
// Role: FullAttention::forward for l > 1 (paramecia-model/src/qwen3_next.rs:2401-2605):
// after a chunk of l tokens is appended, its l queries attend causally over every key
// (query i sees key j iff j <= i + q_offset, q_offset = len - l), GQA group 8, scores
// scaled, clamped to +-100, soft-maxed and applied to V.
//
// Work split: a workgroup owns one KV head, 16 query positions (128 rows = 16 positions
// x 8 heads of the group) and one split of the keys. Its 8 waves each own 16 rows (two
// positions); every 32-key block is dequantized ONCE into fp16 MFMA operand fragments
// in LDS by waves 0-4 and then consumed by all eight waves, so the dequantization cost
// is shared by 128 query rows. Key splits keep 256 workgroups busy; a small kernel
// merges the splits' (m, l, o) partials.
//
// Arithmetic is the decode kernel's (exact fp16 operands, f32 accumulation):
//   QK: A[key][e] = nibble * scale code (an integer <= 945, exact in fp16),
//       B[e][row] = q as fp16 hi and lo parts (two MFMAs into one accumulator),
//       score = d * S1 - dmin * S2 with S2 = sum_j m_j * qsum_j.
//   PV: B[key][e] = (nibble - 8) * scale code * 2^e_d (exact fp16), A[row][key] =
//       p * mantissa(d) as fp16 hi and lo parts; the min term uses A' = p *
//       mantissa(dmin) (hi and lo) against B'[key][j] = m_j * 2^e_dmin, minus A against
//       B''[key][j] = 8 * scale code * 2^e_d, and is subtracted per (row, sub-block) at
//       the end. Centring the nibbles keeps the running PV sums near the size of the
//       output: with nibble * scale alone every value carries its sub-block's offset
//       dmin * m (about 2.5 for N(0,1) rows against outputs near 0.01 at 16k keys), and
//       the f32 rounding of a sum that long then grew with the keys of a split (row
//       errors of 1e-4 of the row at 4k keys per split; about 5e-6 centred).
#include "pkv_mfma_common.hpp"
#include "pkv_prefill_common.hpp"

namespace pkv {

namespace {

// Fp16 operand fragments and tables of one 32-key block of one KV head.
struct DqBlock {
  h8 ka[2][8][64];  // QK A: [tile][step][lane], steps 0-3 low nibbles, 4-7 high
  h4 ka2[2][64];    // S2 A: m codes of sub-blocks 2g, 2g+1
  h8 vb[16][64];    // PV B: [tile T2 = 8h + 2 byte + hl][lane]
  h8 vbm[64];       // min-term B: m_j * 2^e_dmin for columns j < 8
  h8 vbc[64];       // centring B: -8 * sc_j * 2^e_d for columns j < 8
  float kd[kBlk], kdm[kBlk];    // K: d * sl2, dmin * sl2
  float vmd[kBlk], vmdm[kBlk];  // V: mantissas of d and dmin
  _Float16 vsc[8][kBlk], vc[8][kBlk], vm[8][kBlk], vcc[8][kBlk];  // V constants [j][key]
};

struct PfSmem {
  Stage raw[kRaw];
  DqBlock dq[2];  // block i's operands in dq[i & 1] while block i + 1's are built
  float cmin[kPfWaves][16][8];  // per wave: min term [row][j]
};
static_assert(sizeof(PfSmem) <= 160 * 1024, "LDS budget of one workgroup");

// ---- dequantization of one staged block (waves 0-4)

// Waves 0-1: QK A fragments of tile t (the layout of the decode kernel's phase Q).
__device__ __forceinline__ void dq_keys(const Stage &st, DqBlock &D, float sl2, const Masks &MK,
                                        int t, int lane) {
  const int r = lane & 15, g = lane >> 4;
  const int kk = 8 * (r >> 2) + 4 * t + (r & 3);
  const int sw = swz(kk);
  const u4 hd = st.k.hdr[kk];
  const u4 q0 = st.k.nib[8 * kk + ((2 * g) ^ sw)];
  const u4 q1 = st.k.nib[8 * kk + ((2 * g + 1) ^ sw)];
  if (g == 0) {
    D.kd[kk] = h2f(hd.x & 0xFFFF) * sl2;
    D.kdm[kk] = h2f(hd.x >> 16) * sl2;
  }
  uint32_t sc0, sc1, m0, m1;
  scale_min(hd.y, hd.z, hd.w, 2 * g, sc0, m0);
  scale_min(hd.y, hd.z, hd.w, 2 * g + 1, sc1, m1);
  const _Float16 f0 = (_Float16)(float)sc0, f1 = (_Float16)((float)sc1 * 0.0625f);
  const _Float16 c0 = (_Float16)(-1024.0f * (float)sc0), c1 = (_Float16)(-64.0f * (float)sc1);
  const h2 SC0 = {f0, f0}, SC1 = {f1, f1}, C0 = {c0, c0}, C1 = {c1, c1};
  const uint32_t qd[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
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
    D.ka[t][s][lane] = lo;
    D.ka[t][4 + s][lane] = hi;
  }
  D.ka2[t][lane] = h4{(_Float16)(float)m0, (_Float16)(float)m1, (_Float16)0.0f, (_Float16)0.0f};
}

// Waves 2-3: PV B fragments of e-half h (tiles T2 = 8h..8h+7), after their scale tables.
__device__ __forceinline__ void dq_values(const Stage &st, DqBlock &D, const Masks &MK, int h,
                                          int lane) {
  {
    // tables of sub-blocks 4h..4h+3: lane takes key lane % 32, sub-blocks 4h + 2 (lane /
    // 32) + {0, 1}
    const int kk = lane & 31, jp = lane >> 5;
    const u4 vh = st.v.hdr[kk];
    int ed;
    float md;
    split_scale(h2f(vh.x & 0xFFFF), ed, md);
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int j = 4 * h + 2 * jp + jj;
      uint32_t sc, m;
      scale_min(vh.y, vh.z, vh.w, j, sc, m);
      // both nibble forms enter as fp16 1024 + 16 n: (1024 + 16 n) * scp / 16 - 72 scp
      // = (n - 8) scp, exact (72 sc = 8 * 9 sc has at most 10 significant bits)
      const float scp = __builtin_ldexpf((float)sc, ed);
      D.vsc[j][kk] = (_Float16)(scp * 0.0625f);
      D.vc[j][kk] = (_Float16)(-72.0f * scp);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int n = lane & 15, g = lane >> 4;
  uint32_t vq[8];
  const uint32_t *v32 = reinterpret_cast<const uint32_t *>(st.v.nib);
#pragma unroll
  for (int k = 0; k < 8; k += 2) {
    const int R = 8 * g + k;
    const int piece = 4 * h + (n >> 2);
    const int base = 4 * (8 * R + (piece ^ swz(R))) + (n & 3);
    vq[k] = v32[base];
    vq[k + 1] = v32[base + 32];
  }
  const int c = 2 * h + (n >> 3);
  const h8 SL = *reinterpret_cast<const h8 *>(&D.vsc[2 * c][8 * g]);
  const h8 CL = *reinterpret_cast<const h8 *>(&D.vc[2 * c][8 * g]);
  const h8 SH = *reinterpret_cast<const h8 *>(&D.vsc[2 * c + 1][8 * g]);
  const h8 CH = *reinterpret_cast<const h8 *>(&D.vc[2 * c + 1][8 * g]);
#pragma unroll
  for (int byte = 0; byte < 4; ++byte) {
    const uint32_t sel = (uint32_t)byte | (0x0Cu << 8) | ((uint32_t)(4 + byte) << 16) | (0x0Cu << 24);
    h8 blo, bhi;
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      const uint32_t x = __builtin_amdgcn_perm(vq[2 * pp + 1], vq[2 * pp], sel);
      const h2 lo = pk_fma(as_h2(and_or(x << 4, MK.hi, MK.magic)), h2{SL[2 * pp], SL[2 * pp + 1]},
                           h2{CL[2 * pp], CL[2 * pp + 1]});
      const h2 hi = pk_fma(as_h2(and_or(x, MK.hi, MK.magic)), h2{SH[2 * pp], SH[2 * pp + 1]},
                           h2{CH[2 * pp], CH[2 * pp + 1]});
      blo[2 * pp] = lo[0];
      blo[2 * pp + 1] = lo[1];
      bhi[2 * pp] = hi[0];
      bhi[2 * pp + 1] = hi[1];
    }
    D.vb[8 * h + 2 * byte][lane] = blo;
    D.vb[8 * h + 2 * byte + 1][lane] = bhi;
  }
}

// Wave 4: V mantissas and the min-term B fragment.
__device__ __forceinline__ void dq_value_mins(const Stage &st, DqBlock &D, int lane) {
  {
    const int kk = lane & 31, half = lane >> 5;
    const u4 vh = st.v.hdr[kk];
    int ed, em;
    float md, mm;
    split_scale(h2f(vh.x & 0xFFFF), ed, md);
    split_scale(h2f(vh.x >> 16), em, mm);
    (half ? D.vmdm : D.vmd)[kk] = half ? mm : md;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int j = 4 * half + jj;
      uint32_t sc, m;
      scale_min(vh.y, vh.z, vh.w, j, sc, m);
      D.vm[j][kk] = (_Float16)__builtin_ldexpf((float)m, em);
      D.vcc[j][kk] = (_Float16)__builtin_ldexpf(-8.0f * (float)sc, ed);  // exact: |8 sc| <= 504
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int n = lane & 15, g = lane >> 4;
  const h8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
  const h8 bm = *reinterpret_cast<const h8 *>(&D.vm[n & 7][8 * g]);
  const h8 bc = *reinterpret_cast<const h8 *>(&D.vcc[n & 7][8 * g]);
  D.vbm[lane] = n < 8 ? bm : zero8;
  D.vbc[lane] = n < 8 ? bc : zero8;
}

// The 6 loads of one tensor of one block: issued by one wave, so that its vmcnt counts
// exactly its own loads.
__device__ __forceinline__ void issue_tensor(TensorStage *ts, const LoadPlan &P, u4s rsrc,
                                             uint32_t boff) {
  const uint32_t n0 = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)((PKV_LDS void *)&ts->nib[0]));
  const uint32_t h0 = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)((PKV_LDS void *)&ts->hdr[0]));
  uint32_t saved;
  asm volatile(
      "s_nop 4\n\t"  // VALU-written SGPRs (v_readfirstlane) read by VMEM: 5 wait states
      "s_mov_b32 %[sv], m0\n\t"
      "s_mov_b32 m0, %[n0]\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o0], %[rs], 0 offen lds\n\t"
      "s_add_u32 m0, %[n0], 0x400\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o1], %[rs], 0 offen lds\n\t"
      "s_add_u32 m0, %[n0], 0x800\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o2], %[rs], 0 offen lds\n\t"
      "s_add_u32 m0, %[n0], 0xc00\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o3], %[rs], 0 offen lds\n\t"
      "s_mov_b32 m0, %[h0]\n\ts_nop 0\n\t"
      "buffer_load_dword %[p0], %[rs], 0 offen lds\n\t"
      "s_add_u32 m0, %[h0], 0x100\n\ts_nop 0\n\t"
      "buffer_load_dword %[p1], %[rs], 0 offen lds\n\t"
      "s_mov_b32 m0, %[sv]"
      : [sv] "=&s"(saved)
      : [n0] "s"(n0), [h0] "s"(h0), [o0] "v"(P.nib[0] + boff), [o1] "v"(P.nib[1] + boff),
        [o2] "v"(P.nib[2] + boff), [o3] "v"(P.nib[3] + boff), [p0] "v"(P.hdr[0] + boff),
        [p1] "v"(P.hdr[1] + boff), [rs] "s"(rsrc)
      : "memory", "scc");
}

__global__ __launch_bounds__(kPfThreads) void q4k_prefill_kernel(PrefillArgs a) {
  __shared__ PfSmem sm;
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
  const uint32_t span = a.seq_k > 0 ? (uint32_t)(a.seq_k - 1) * rs_t + 144u : 0u;
  const u4s rk = make_rsrc(kbase, span), rv = make_rsrc(vbase, span);
  const LoadPlan P = make_plan(lane, rs_t);
  const uint32_t bbytes = kBlk * rs_t;
  const bool loader = wave == 5 || wave == 6;
  auto issue = [&](int i) {  // raw block i of this workgroup into stage i % kRaw
    if (wave == 5) issue_tensor(&sm.raw[i % kRaw].k, P, rk, (uint32_t)(kb0 + i) * bbytes);
    if (wave == 6) issue_tensor(&sm.raw[i % kRaw].v, P, rv, (uint32_t)(kb0 + i) * bbytes);
  };
  if (loader) {
    if (nb > 0) issue(0);
    if (nb > 1) issue(1);
  }

  // ---- q operands of this wave's 16 rows (row n: position pw + n / 8, head 8 kvg + n % 8)
  h8 qbh[8], qbl[8];
  h4 q2h = {0, 0, 0, 0}, q2l = {0, 0, 0, 0};
  {
    const int pos = pw + (n >> 3);
    const bool ok = pos < a.l;
    const float *qrow = a.q + (((int64_t)b * a.l + (ok ? pos : 0)) * 16 + 8 * kvg + (n & 7)) * 256 + 64 * g;
    constexpr int perm[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    float qsum[2] = {0.0f, 0.0f};
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      // rows past the chunk read position 0 and are never stored
      const float4 r0 = *reinterpret_cast<const float4 *>(qrow + 32 * (st >> 2) + 8 * (st & 3));
      const float4 r1 = *reinterpret_cast<const float4 *>(qrow + 32 * (st >> 2) + 8 * (st & 3) + 4);
      const float v8[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
#pragma unroll
      for (int k = 0; k < 8; ++k) qsum[st >> 2] += v8[k];
#pragma unroll
      for (int slot = 0; slot < 8; ++slot) {
        const float qv = v8[perm[slot]];
        const _Float16 hi = (_Float16)qv;
        qbh[st][slot] = hi;
        qbl[st][slot] = (_Float16)(qv - (float)hi);
      }
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const _Float16 hi = (_Float16)qsum[t];
      q2h[t] = hi;
      q2l[t] = (_Float16)(qsum[t] - (float)hi);
    }
  }

  f4 acc[16];
#pragma unroll
  for (int T2 = 0; T2 < 16; ++T2) acc[T2] = f4{0.f, 0.f, 0.f, 0.f};
  f4 accm = {0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, lsum = 0.0f;
  const Masks MK = {vconst(0x000F000Fu), vconst(0x00F000F0u), vconst(0x64006400u)};
  // position of this lane's row (n): the causal limit of its keys
  const int64_t myq = (int64_t)pw + (n >> 3);
  const int64_t klim = a.causal ? myq + a.q_offset : (int64_t)1 << 62;

  // Waves 0-4 build the fp16 operands of block i + 1 while every wave runs the MFMAs of
  // block i (waves 0-3 before them, wave 4 right after issuing its QK MFMAs): one
  // barrier per block. Raw stages rotate over kRaw = 3 (blocks i + 1 and
  // i + 2 in flight or landed while block i + 3 is issued).
  auto dequant = [&](int blk) {
    const Stage &st = sm.raw[blk % kRaw];
    DqBlock &Dn = sm.dq[blk & 1];
    if (wave < 2)
      dq_keys(st, Dn, a.sl2, MK, wave, lane);
    else if (wave < 4)
      dq_values(st, Dn, MK, wave - 2, lane);
  };
  // Wave 4 builds the small min tables of block i + 1 (a few LDS round trips, little
  // VALU) while its QK MFMAs of block i run, ahead of wave 0, which shares its SIMD: at
  // the top of the block they put this wave's MFMAs after wave 0's dequantization.
  auto dequant_mins = [&](int blk) {
    __builtin_amdgcn_s_setprio(2);
    dq_value_mins(sm.raw[blk % kRaw], sm.dq[blk & 1], lane);
    __builtin_amdgcn_s_setprio(0);
  };
  if (nb > 0) {
    if (loader) {  // block 0 landed (block 1 may still fly)
      if (nb > 1)
        asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    if (loader && nb > 2) issue(2);
    dequant(0);
    if (wave == 4) dequant_mins(0);
  }
  for (int i = 0; i < nb; ++i) {
    if (loader && i + 1 < nb) {  // block i + 1 landed (block i + 2 may still fly)
      if (i + 2 < nb)  // the 6 loads of block i + 2 may stay in flight
        asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    // operands of block i ready; raw block i + 1 visible; block i - 1's operands and
    // block i's raw stage no longer read
    __syncthreads();
    if (loader && i + 3 < nb) issue(i + 3);
    if (i + 1 < nb) dequant(i + 1);
    const DqBlock &D = sm.dq[i & 1];

    // ---- QK (two tiles of 16 keys), rows = this wave's 16 query rows; keys kk of the
    // block at or past nlim are masked (past the cache, or past this row's causal limit)
    const int64_t key0 = (int64_t)(kb0 + i) * kBlk;
    int64_t lim = a.seq_k < klim + 1 ? a.seq_k : klim + 1;
    lim -= key0;
    const int nlim = lim < 0 ? 0 : (lim > kBlk ? kBlk : (int)lim);
    float sc8[8];
    // four independent accumulator chains (tile x q part), interleaved so that the
    // MFMA pipe never waits for the previous result of the same chain
    f4 s1h[2], s1l[2], s2[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) s1h[t] = s1l[t] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const h8 A = D.ka[t][s][lane];
        s1h[t] = mfma32(A, qbh[s], s1h[t]);
        s1l[t] = mfma32(A, qbl[s], s1l[t]);
      }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const h4 A2 = D.ka2[t][lane];
      s2[t] = mfma16(A2, q2h, f4{0.f, 0.f, 0.f, 0.f});
      s2[t] = mfma16(A2, q2l, s2[t]);
    }
    if (wave == 4 && i + 1 < nb) {
      __builtin_amdgcn_sched_barrier(0);  // the MFMAs above go out first
      dequant_mins(i + 1);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const f4 s1 = s1h[t] + s1l[t];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int kk = 8 * g + 4 * t + ii;
        float sc = D.kd[kk] * s1[ii] - D.kdm[kk] * s2[t][ii];
        sc = fminf(fmaxf(sc, -kClampL2), kClampL2);
        sc8[4 * t + ii] = kk < nlim ? sc : -INFINITY;
      }
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
      for (int T2 = 0; T2 < 16; ++T2)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) acc[T2][ii] *= ai[ii];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) accm[ii] *= ai[ii];
    }
    float p[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      // a row with no visible key so far keeps m_run = -inf: its p are 0
      p[k] = (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(sc8[k] - m_run);
      lsum += p[k];
    }
    // ---- PV: A rows = query rows, keys 8g..8g+7. The weights p * mantissa enter as
    // fp16 hi and lo parts (~22 bits): one fp16 rounding of a weight (2^-12 relative)
    // times a value of an outlier channel would exceed the attention tolerance.
    uint32_t wa[4], wl[4], wm[4], wml[4];
#pragma unroll
    for (int k2 = 0; k2 < 4; ++k2) {
      const float x0 = p[2 * k2] * D.vmd[8 * g + 2 * k2];
      const float x1 = p[2 * k2 + 1] * D.vmd[8 * g + 2 * k2 + 1];
      const float y0 = p[2 * k2] * D.vmdm[8 * g + 2 * k2];
      const float y1 = p[2 * k2 + 1] * D.vmdm[8 * g + 2 * k2 + 1];
      wa[k2] = as_u(h2{(_Float16)x0, (_Float16)x1});
      wl[k2] = fp16_sub2(x0, x1, wa[k2]);
      wm[k2] = as_u(h2{(_Float16)y0, (_Float16)y1});
      wml[k2] = fp16_sub2(y0, y1, wm[k2]);
    }
    const h8 A = __builtin_bit_cast(h8, u4{wa[0], wa[1], wa[2], wa[3]});
    const h8 Al = __builtin_bit_cast(h8, u4{wl[0], wl[1], wl[2], wl[3]});
    const h8 Am = __builtin_bit_cast(h8, u4{wm[0], wm[1], wm[2], wm[3]});
    const h8 Aml = __builtin_bit_cast(h8, u4{wml[0], wml[1], wml[2], wml[3]});
#pragma unroll
    for (int T2 = 0; T2 < 16; ++T2) {
      const h8 B = D.vb[T2][lane];
      acc[T2] = mfma32(A, B, acc[T2]);
      acc[T2] = mfma32(Al, B, acc[T2]);
    }
    const h8 Bm = D.vbm[lane], Bc = D.vbc[lane];
    accm = mfma32(Am, Bm, accm);
    accm = mfma32(Aml, Bm, accm);
    accm = mfma32(A, Bc, accm);
    accm = mfma32(Al, Bc, accm);
  }

  // ---- epilogue: row sums, min-term subtraction, then output or partial
  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
  float(*cmin)[8] = sm.cmin[wave];
  if (n < 8) {
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) cmin[4 * g + ii][n] = accm[ii];  // rows 4g+ii, column j=n
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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
      for (int T2 = 0; T2 < 16; ++T2) {
        const int e = tile_e(T2, n);
        orow[e] = (acc[T2][ii] - cmin[row][e >> 5]) * inv;
      }
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
      for (int T2 = 0; T2 < 16; ++T2) {
        const int e = tile_e(T2, n);
        prow[16 * T2 + n] = acc[T2][ii] - cmin[row][e >> 5];
      }
      if (n == 0) {
        prow[256] = mrow[ii];
        prow[257] = lrow[ii];
      }
    }
  }
}

}  // namespace

int launch_prefill_mfma(const AttnArgs &a, Workspace &ws, hipStream_t s) {
  if (a.quant != PKV_QUANT_Q4K || a.head_dim != 256 || a.num_heads != 16 ||
      a.num_kv_heads != 2 || a.l < 2)
    return PKV_ERR_UNSUPPORTED;
  if (a.rs.t >= (1 << 24) || a.seq_k >= (1 << 24) ||
      (uint64_t)a.seq_k * (uint64_t)a.rs.t >= (1ull << 32))
    return PKV_ERR_UNSUPPORTED;
  PrefillArgs d;
  const int rc = prefill_plan(a, a.scale * kLog2e, ws, d);
  if (rc) return rc;
  hipLaunchKernelGGL(q4k_prefill_kernel, dim3((unsigned)(d.ntiles * d.ngroups)),
                     dim3(kPfThreads), 0, s, d);
  PKV_HIP(hipGetLastError());
  return prefill_merge(d, a.batch, s);
}

}  // namespace pkv
