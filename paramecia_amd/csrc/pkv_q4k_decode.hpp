// MFMA decode attention over a Q4K cache for the Qwen3-Next full-attention shape
// (16 query heads, 2 KV heads, head_dim 256), gfx950.
//
// Role: the dequant-fused attention of the reference's flash_attn_q8 path
// (paramecia-model/src/ops.rs:756-792, called at qwen3_next.rs:2531-2561) and the CPU
// SDPA it falls back to (qwen3_next.rs:2580-2605), for a decode step (one query).
//
// Work split: split-K over 32-key blocks. A workgroup of 8 waves (two per SIMD, so each
// SIMD always has a second wave to issue while one waits) owns a contiguous block
// range; waves 2s and 2s+1 take KV heads 0 and 1 of the same blocks, so the two halves
// of a token's 288-byte K (and V) rows are read together. Each wave streams its blocks
// through two LDS stages with buffer_load ... lds. With several segments (the sequences
// of a batched step) the launch's blocks form one line that the workgroups split evenly
// (stream-K): a workgroup whose range crosses a segment boundary runs one pass per
// segment, each with its own partial. Waves 0-3 of the first workgroups also quantize
// the new token's rows for a fused decode step (bit-exact Q4K).
//
// Arithmetic (per KV head, per 16 keys, MFMA f32_16x16x32_f16):
//   QK: A[key][e] = nibble * sub-block scale code, an integer <= 945 built exactly in
//       fp16 from the packed byte with the 1024-offset trick and one v_pk_fma;
//       B[e][col] = q split into fp16 hi/lo parts: columns 0-7 are the hi parts of the
//       group's 8 heads, 8-15 the lo parts, so hi+lo recover q to ~22 bits.
//       score = d * S1 - dmin * S2 with S2 = sum_j m_j * qsum_j (a 16x16x16 MFMA).
//   PV: B[key][e] = nibble * scale code * 2^e_d (exact fp16, e_d = exponent of d),
//       A[head][key] = p * mantissa(d): rows 0-7 its fp16 hi part, rows 8-15 the lo
//       remainder (rows h and 8 + h are summed after the loop, ~22 bits). The min term
//       A'[head][key] = p * mantissa(dmin) (hi and lo rows alike) against
//       B'[key][j] = m_j * 2^e_dmin.
//   All accumulation is f32. Softmax runs in base 2 with the 1/sqrt(d) scale folded
//   in, scores clamped to [-100, 100] (in natural-log units) as the reference does.
//   The running max is raised only when a block exceeds it by 2^8, so the
//   accumulators are rarely rescaled.
// Include-only: the kernel template and its launch plan, instantiated by
// pkv_attn_mfma.hip (kPrep = false) and pkv_attn_mfma_prep.hip (kPrep = true).
#pragma once
#include <cstdlib>

#include "pkv_decode_split.hpp"
#include "pkv_mfma_common.hpp"
#include "pkv_q4k_lanes.hpp"
#include "pkv_prep_common.hpp"

namespace pkv {

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;  // two waves per SIMD
constexpr int kMainWGs = 256;
// Quantize-only workgroups in front of a one-row fused launch of nwg decode workgroups
// (the in-launch combine's full grid has none): 4 when the CUs have room for them.
__host__ __device__ constexpr int kQuantFront(bool one, bool fused, int nwg) {
  return one && fused && nwg <= kMainWGs - 4 ? 4 : 0;
}
constexpr float kLazy = 8.0f;  // log2 headroom of the running max before a rescale
constexpr int kPieceGap = 6;   // virtual blocks before each segment after the first

// Kernel arguments: the fields shared by every launch, then the segment table sized at
// compile time (one segment for a single cache of batch 1, kMaxSegs otherwise), so that the
// common launch carries about 200 bytes of arguments instead of the 1.5 KB of the full
// table.
struct DecodeArgsBase {
  int nseg, nwg;  // segments (or paged sequences), workgroups
  int vq, vr;     // workgroup w's range on the virtual block line starts at
                  // w vq + min(w, vr) and holds vq + (w < vr) blocks
  int64_t rs_t, rs_h;
  float sl2;                   // scale * log2(e)
  const float *q;              // [nseg][16][256]
  const float *k_new, *v_new;  // [nseg][2][256] or null (fused decode step)
  float *part;                 // [nwg][16][kPartRow]
  float2 *ml;                  // [nwg][16] running max and sum
  float *dq;  // [nseg][4][256] dequantized new rows (K kv0, K kv1, V kv0, V kv1)
  // q/k preparation of a decode step from projection outputs (q_norm, k_norm, rope at
  // each segment's new position); used by the kPrep instantiation only
  DecodePrep prep;
  float *q_out;  // [nseg][16][256] prepared q, for the combine
  unsigned *status;  // the device status word (pkv_device_status)
  // Fused step: the new rows of nnew output rows (4 nnew rows: K and V of each KV
  // head), at row t_new of segment i, or for paged sequences at row len of their page
  int nnew;
  // In-launch combine (one segment): ncomb combiner workgroups follow the nwg decode
  // workgroups in the grid and merge the partials as they arrive; 0 = the separate
  // combine kernel. `words` are the control words of the workspace's fused region (see
  // tail_combine), part / ml then point into that region.
  int ncomb;
  uint32_t *words;
  float *out;  // [16][256]: the combiners' output row
};
template <int kSegs>
struct DecodeArgsT : DecodeArgsBase {
  DecodeSeg seg[kSegs];
};
// Paged sequences with device page lists (kSegs == 0, the paged Q4K decode): output row i
// attends to len keys held in pages[0..npg) of the pool's planes. Its segment j (page j)
// sits on the virtual block line at vstart + j * pstride (pstride = blocks per page + the
// gap), with the blocks of the keys it holds, or one virtual block for a sequence
// without keys (a fused step's first token); kfirst numbers its segment 0 among all
// segments of the launch. The fused step's new row of sequence i is row len of page
// pages[len >> page_lg].
struct PagedSeqArg {
  const int32_t *pages;
  int64_t len;
  int vstart, npg, kfirst, pad;
};
template <>
struct DecodeArgsT<0> : DecodeArgsBase {
  PagedSeqArg pq[kMaxSegs];
  uint8_t *kplane, *vplane;
  int64_t page_bytes;
  int page_lg, pstride;
  int nsegs;  // segments of the launch
};

// Per-wave tables rebuilt for every 32-key block.
struct WaveTab {
  float kd[kBlk], kdm[kBlk];                        // epilogue exchange (cmin); see below
  float vmd[kBlk], vmdm[kBlk];                      // V: mantissas of d and dmin
  _Float16 vsc[8][kBlk], vc[8][kBlk], vm[8][kBlk];  // V: fp16 constants [j][key]
};

// LDS of one workgroup. Each wave owns stage buffers st[w][0], st[w][1] (adjacent, so
// both are reached from one base register with immediate offsets) and a table area;
// before its first refill of st[w][1] a wave stages its KV head's q rows there, and the
// quantizer scratch of the quantizing waves 0-3 overlaps their tables (used before their
// block loops or once all four have left them). The merge area
// reuses the first stage buffers once every wave has left the loop. Stages are always addressed by
// indexing this array: a pointer chosen at run time between two stages loses its LDS
// address space, and the generic (flat) loads it then compiles to wait on every
// outstanding buffer load, including the prefetch of the next block.
struct Smem {
  union {
    struct {
      Stage st[kWaves][2];
      union {
        WaveTab tab[kWaves];
        struct {
          Q4kScratch scr;
          __attribute__((aligned(16))) float prow[256];  // k_norm / rope of a K row
          float pm;
        } quant;
      } t;
    } run;
    struct {
      float4 o[kWaves][16][2][16];  // [wave][T2][row group g][n]: rows 4g..4g+3, scaled
    } merge;
  };
};
// The quantizing waves' barrier counter is tab[1].kd[0]: no wave writes a kd table
// before the epilogue's first workgroup barrier (the prepared-q constants are staged in
// vc / vm), and the quantizer scratch stays within tab[0].
static_assert(sizeof(Smem{}.run.t.quant) <= sizeof(WaveTab), "quantizer scratch within tab[0]");
static_assert(offsetof(decltype(Smem{}.run.t.quant), prow) >= sizeof(Q4kScratch) &&
                  sizeof(Smem{}.run.t.quant) <= 4 * sizeof(WaveTab),
              "quantizer scratch within the tables of the quantizing waves 0-3");
static_assert(sizeof(float4[kWaves][16][2][16]) <= sizeof(Stage[kWaves]),
              "merge area within the first stage buffers");
static_assert(24 <= kBlk, "m, l and f * l of 8 heads fit a wave's vmd table");
static_assert(sizeof(Smem) <= 160 * 1024, "LDS budget of one workgroup");

// Stage this wave's KV head's 8 q rows (8 KB, contiguous in q) into LDS: eight
// dwordx4 loads, lane l of load j moving bytes 1024 j + 16 l of q to LDS byte
// kQRow j + 16 l. The 16-byte pad per row puts the rows' reads in build_q (one row per
// lane, same column) on different banks.
constexpr int kQRow = 1040;  // bytes per staged q row (256 floats + 16 bytes of pad)
static_assert(8 * kQRow <= (int)sizeof(Stage), "q rows fit one stage");
__device__ __forceinline__ void issue_q(void *dst_lds, u4s rq, uint32_t lane16) {
  const uint32_t dst = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)((PKV_LDS void *)dst_lds));
  uint32_t saved;
  asm volatile(
      "s_nop 4\n\t"  // VALU-written SGPRs (v_readfirstlane) read by VMEM: 5 wait states
      "s_mov_b32 %[sv], m0\n\t"
      "s_mov_b32 m0, %[d]\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o0], %[rq], 0 offen lds\n\t"
      "s_add_u32 m0, %[d], 0x410\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o1], %[rq], 0 offen lds\n\t"
      "s_add_u32 m0, %[d], 0x820\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o2], %[rq], 0 offen lds\n\t"
      "s_add_u32 m0, %[d], 0xc30\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o3], %[rq], 0 offen lds\n\t"
      "s_add_u32 m0, %[d], 0x1040\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o4], %[rq], 0 offen lds\n\t"
      "s_add_u32 m0, %[d], 0x1450\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o5], %[rq], 0 offen lds\n\t"
      "s_add_u32 m0, %[d], 0x1860\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o6], %[rq], 0 offen lds\n\t"
      "s_add_u32 m0, %[d], 0x1c70\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o7], %[rq], 0 offen lds\n\t"
      "s_mov_b32 m0, %[sv]"
      : [sv] "=&s"(saved)
      : [d] "s"(dst), [o0] "v"(lane16), [o1] "v"(lane16 + 1024u), [o2] "v"(lane16 + 2048u),
        [o3] "v"(lane16 + 3072u), [o4] "v"(lane16 + 4096u), [o5] "v"(lane16 + 5120u),
        [o6] "v"(lane16 + 6144u), [o7] "v"(lane16 + 7168u), [rq] "s"(rq)
      : "memory", "scc");
}

struct WaveState {
  f4 acc[16];  // PV accumulators, tile T = 8h + 2*byte + hl
  f4 accm;     // min-term accumulator
  float m_run, lsum;
};

struct QKOut {
  f4 s1[2], s2[2];  // per 16-key tile: sum_e (n*sc)_e q_e and sum_j m_j qsum_j
};

// Lane constants of the K scale decode. Lane group g uses sub-blocks 2g and 2g + 1,
// whose 6-bit scale and min codes sit in bytes 2(g & 1), 2(g & 1) + 1 of the header's
// words s0 (scales 0-3), s1 (mins 0-3) and, for sub-blocks 4-7, s2 (low 4 bits) with
// the top two bits in s0 / s1 (get_scale_min_k4). v_perm puts header byte b of s2 (or
// s0 / s1 for g < 2) in the low byte and byte b of s0 / s1 in the high byte of each
// 16-bit half; the masks then keep the code's low bits in place and move bits 6-7 of
// the high byte down to bits 4-5, and the 0x6400 exponent makes each half the fp16
// value 1024 + code.
struct KScaleSel {
  uint32_t perm;  // v_perm selector: S0 = s0 or s1, S1 = s2
  uint32_t lo;    // low code bits kept in place: 0x3F (g < 2) or 0x0F per half
  uint32_t up;    // bits 4-5 taken from bits 14-15 of each half (g >= 2)
  uint32_t msh;   // right shift of the min codes' low bits: 0 (g < 2) or 4
};
__device__ __forceinline__ KScaleSel make_kscale_sel(int g) {
  const uint32_t b = 2u * (uint32_t)(g & 1);
  KScaleSel s;
  if (g < 2) {
    s.perm = (4u + b) | (0x0Cu << 8) | ((5u + b) << 16) | (0x0Cu << 24);
    s.lo = 0x003F003Fu;
    s.up = 0u;
    s.msh = 0u;
  } else {
    s.perm = b | ((4u + b) << 8) | ((b + 1u) << 16) | ((5u + b) << 24);
    s.lo = 0x000F000Fu;
    s.up = 0x00300030u;
    s.msh = 4u;
  }
  return s;
}
// {1024 + code(2g), 1024 + code(2g + 1)} as fp16 halves: the scale codes from (s0, s2),
// the min codes from (s1, s2)
__device__ __forceinline__ uint32_t kcode_pair(uint32_t sx, uint32_t s2, uint32_t sh,
                                               const KScaleSel &ks, uint32_t magic) {
  const uint32_t P = __builtin_amdgcn_perm(sx, s2, ks.perm);
  return and_or(P >> sh, ks.lo, and_or(P >> 10, ks.up, magic));
}

// Header and K words of a staged block, read together right after the stage's vmcnt
// wait so that their LDS latencies overlap instead of each one stalling its phase. The
// wait covers every word of the stage: on gfx950 a buffer_load ... lds counts in vmcnt
// until its data is in LDS, and the only vector-memory instructions between a stage's
// issue and its wait are the next stage's 12 loads (checked word by word against
// global memory in both the immediate and the pipelined pattern).
struct BlockWords {
  u4 khd[2], kq0[2], kq1[2];  // phase Q: header and nibble pieces of key kk(r) per tile
  uint32_t hx[8];             // phase S: {d, dmin} of keys 8g..8g+7
  u4 vhd;                     // phase P: V header of key lane % 32
};
__device__ __forceinline__ void load_block_words(const Stage &st, int lane, BlockWords &W) {
  const int r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int kk = 8 * (r >> 2) + 4 * t + (r & 3);
    const int sw = swz(kk);
    W.khd[t] = st.k.hdr[kk];
    W.kq0[t] = st.k.nib[8 * kk + ((2 * g) ^ sw)];
    W.kq1[t] = st.k.nib[8 * kk + ((2 * g + 1) ^ sw)];
  }
  const uint32_t *hdr32 = reinterpret_cast<const uint32_t *>(st.k.hdr);
#pragma unroll
  for (int k = 0; k < 8; ++k) W.hx[k] = hdr32[4 * (8 * g + k)];
  W.vhd = st.v.hdr[lane & 31];
}

// Phase Q: K rows of a staged block -> raw QK sums.
// Lane (r, g) feeds key kk(r) of tile t with sub-blocks 2g (low nibbles) and 2g+1
// (high nibbles); its min codes m_2g, m_2g+1 form the A operand of the S2 product.
__device__ __forceinline__ void phase_q(const BlockWords &W, const h8 *qb, h4 q2, const Masks &MK,
                                        const KScaleSel &ks, QKOut &o) {
  // pk_fma constants: {1024 + sc0, 1024 + sc1} -> {sc0, sc1 / 16}; then the offsets
  // {-1024 sc0, -64 sc1} of the two nibble forms (1024 + n, 1024 + 16 n)
  const h2 ksc = {(_Float16)1.0f, (_Float16)0.0625f}, kcc = {(_Float16)-1024.0f, (_Float16)-64.0f};
  const h2 kneg = {(_Float16)-1024.0f, (_Float16)-1024.0f};
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const u4 hd = W.khd[t], q0 = W.kq0[t], q1 = W.kq1[t];
    const h2 SC = pk_fma(as_h2(kcode_pair(hd.y, hd.w, 0u, ks, MK.magic)), ksc, kcc);
    const h2 CC = SC * kneg;
    const h2 MM = as_h2(kcode_pair(hd.z, hd.w, ks.msh, ks, MK.magic)) + kneg;
    const h2 SC0 = __builtin_shufflevector(SC, SC, 0, 0), SC1 = __builtin_shufflevector(SC, SC, 1, 1);
    const h2 C0 = __builtin_shufflevector(CC, CC, 0, 0), C1 = __builtin_shufflevector(CC, CC, 1, 1);
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
    const h4 a2 = {MM[0], MM[1], (_Float16)0.0f, (_Float16)0.0f};
    o.s1[t] = s1;
    o.s2[t] = mfma16(a2, q2, f4{0.f, 0.f, 0.f, 0.f});
  }
}

// d * s1 - dmin * s2 with the fp16 pair {d, dmin} of a header dword (one rounded product,
// then one fma). s1 and s2 are MFMA results: written in C, so that the compiler places the
// wait states an MFMA result needs before a VALU reads it (it cannot for inline asm).
__device__ __forceinline__ float hdr_dot(uint32_t hx, float s1, float s2) {
#pragma clang fp contract(off)
  const h2 dd = as_h2(hx);
  const float t = (float)dd[0] * s1;
  return __builtin_fmaf(-(float)dd[1], s2, t);
}

// Phase S: scores (log2 units) and the online softmax; p[k] for key 8g + k, head n % 8.
// Keys at or past nvalid (only in a partial last block) are masked.
// Scores stay in q.k units here (the running max too); sl2 = scale * log2(e) enters
// the exponents, and clamp / lazy are the +-100-nat clamp and the rescale headroom in
// those units.
__device__ __forceinline__ void phase_s(const BlockWords &W, const QKOut &o, WaveState &S,
                                        int nvalid, float sl2, float clamp, float lazy, int lane,
                                        float p[8]) {
  const int g = lane >> 4;
  float sc8[8];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // key 8g + 4t + i: this column's part (hi or lo of q); the other part sits 8 lanes
      // away. d and dmin enter as fp16 (v_fma_mix).
      const float part = hdr_dot(W.hx[4 * t + i], o.s1[t][i], o.s2[t][i]);
      const float sc = part + ror8(part);
      sc8[4 * t + i] = __builtin_amdgcn_fmed3f(sc, -clamp, clamp);
    }
  if (nvalid < kBlk) {
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (8 * g + k >= nvalid) sc8[k] = -INFINITY;
  }
  float bm = sc8[0];
#pragma unroll
  for (int k = 1; k < 8; ++k) bm = fmaxf(bm, sc8[k]);
  bm = xmax32(xmax16(bm));
  if (S.m_run == -INFINITY) {
    // first block with a valid key: nothing accumulated yet, no rescale
    S.m_run = bm;
  } else if (__any(bm > S.m_run + lazy)) {
    const float m_new = fmaxf(S.m_run, bm);
    const float alpha = (S.m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f((S.m_run - m_new) * sl2);
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
  const float nm = -S.m_run * sl2;  // finite: every block has a valid key
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    p[k] = __builtin_amdgcn_exp2f(fmaf(sc8[k], sl2, nm));
    S.lsum += p[k];
  }
}

// Lane constants of the V table build: lane l takes key l % 32 and sub-blocks
// 4u..4u+3 (u = l / 32), whose codes are bytes 0-3 of s0 / s1 (u = 0) or the low 4 bits
// of s2 with bits 6-7 of s0 / s1 above them (u = 1, get_scale_min_k4).
struct VScaleSel {
  uint32_t sh, ma, mb;
};
__device__ __forceinline__ VScaleSel make_vscale_sel(int lane) {
  const bool u = lane >= 32;
  return VScaleSel{u ? 2u : 0u, u ? 0x30303030u : 0x3F3F3F3Fu, u ? 0x0F0F0F0Fu : 0u};
}

// Phase P: V header tables, PV A/B operands and MFMAs, min term.
__device__ __forceinline__ void phase_p(const Stage &st, const BlockWords &W, WaveState &S,
                                        WaveTab &T, const float p[8], const Masks &MK,
                                        const VScaleSel &vs, int lane) {
  const int n = lane & 15, g = lane >> 4;
  // V header -> constant tables. The four codes of a lane come out as bytes; the pairs
  // (4u, 4u+2) and (4u+1, 4u+3) become fp16 1024 + code, and one v_pk_fma each gives
  // sc * 2^e_d (sc * 2^(e_d - 4) for the high-nibble sub-blocks), exact in fp16 for
  // e_d in [-20, 0]; the offsets are -1024 times those.
  {
    const int kk = lane & 31, u = lane >> 5;
    const u4 vh = W.vhd;
    int ed, em;
    float md, mm;
    split_scale(h2f(vh.x & 0xFFFF), ed, md);
    split_scale(h2f(vh.x >> 16), em, mm);
    (u ? T.vmdm : T.vmd)[kk] = u ? mm : md;
    const uint32_t sc4 = and_or(vh.y >> vs.sh, vs.ma, vh.w & vs.mb);
    const uint32_t m4 = and_or(vh.z >> vs.sh, vs.ma, (vh.w >> 4) & vs.mb);
    const _Float16 e1 = __builtin_amdgcn_ldexph((_Float16)1.0f, ed);
    const _Float16 n1 = __builtin_amdgcn_ldexph((_Float16)-1024.0f, ed);
    const _Float16 e4 = __builtin_amdgcn_ldexph((_Float16)0.0625f, ed);
    const _Float16 n4 = __builtin_amdgcn_ldexph((_Float16)-64.0f, ed);
    const _Float16 em1 = __builtin_amdgcn_ldexph((_Float16)1.0f, em);
    const _Float16 nm1 = __builtin_amdgcn_ldexph((_Float16)-1024.0f, em);
    const h2 kneg = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    const h2 se = pk_fma(as_h2(and_or(sc4, 0x00FF00FFu, MK.magic)), h2{e1, e1}, h2{n1, n1});
    const h2 so = pk_fma(as_h2(and_or(sc4 >> 8, 0x00FF00FFu, MK.magic)), h2{e4, e4}, h2{n4, n4});
    const h2 me = pk_fma(as_h2(and_or(m4, 0x00FF00FFu, MK.magic)), h2{em1, em1}, h2{nm1, nm1});
    const h2 mo = pk_fma(as_h2(and_or(m4 >> 8, 0x00FF00FFu, MK.magic)), h2{em1, em1}, h2{nm1, nm1});
    const h2 ce = se * kneg, co = so * kneg;
    const int j = 4 * u;
    T.vsc[j][kk] = se[0];
    T.vsc[j + 2][kk] = se[1];
    T.vsc[j + 1][kk] = so[0];
    T.vsc[j + 3][kk] = so[1];
    T.vc[j][kk] = ce[0];
    T.vc[j + 2][kk] = ce[1];
    T.vc[j + 1][kk] = co[0];
    T.vc[j + 3][kk] = co[1];
    T.vm[j][kk] = me[0];
    T.vm[j + 2][kk] = me[1];
    T.vm[j + 1][kk] = mo[0];
    T.vm[j + 3][kk] = mo[1];
  }
  // V rows, transposed: dword n & 3 of nibble piece 4h + n / 4 of keys 8g..8g+7. Rows
  // 2i and 2i+1 share their swizzle, so each pair is one ds_read2 (128 bytes apart).
  uint32_t vq[2][8];
  const uint32_t *v32 = reinterpret_cast<const uint32_t *>(st.v.nib);
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int k = 0; k < 8; k += 2) {
      const int R = 8 * g + k;
      const int piece = 4 * h + (n >> 2);
      const int base = 4 * (8 * R + (piece ^ swz(R))) + (n & 3);
      vq[h][k] = v32[base];
      vq[h][k + 1] = v32[base + 32];
    }
  // A: rows 0-7 the fp16 hi parts of p * mant(d), rows 8-15 the lo remainders (the two
  // row halves are summed after the loop); Am likewise for p * mant(dmin). One fp16
  // rounding of a weight (2^-12 relative) times a value of an outlier channel would
  // exceed the attention tolerance; hi + lo keeps ~22 bits.
  // Both parts are fp16(x - c) with c = fp16(x) masked to zero on the hi rows.
  const uint32_t lo_mask = n >= 8 ? 0xFFFFFFFFu : 0u;
  uint32_t aw[4], amw[4];
#pragma unroll
  for (int kp = 0; kp < 4; ++kp) {
    const float x0 = p[2 * kp] * T.vmd[8 * g + 2 * kp], x1 = p[2 * kp + 1] * T.vmd[8 * g + 2 * kp + 1];
    const float y0 = p[2 * kp] * T.vmdm[8 * g + 2 * kp], y1 = p[2 * kp + 1] * T.vmdm[8 * g + 2 * kp + 1];
    const uint32_t cx = as_u(h2{(_Float16)x0, (_Float16)x1}) & lo_mask;
    const uint32_t cy = as_u(h2{(_Float16)y0, (_Float16)y1}) & lo_mask;
    aw[kp] = fp16_sub2(x0, x1, cx);
    amw[kp] = fp16_sub2(y0, y1, cy);
  }
  const h8 A = __builtin_bit_cast(h8, u4{aw[0], aw[1], aw[2], aw[3]});
  const h8 Am = __builtin_bit_cast(h8, u4{amw[0], amw[1], amw[2], amw[3]});
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
  // min term: C'[row][j] += sum_k Am[row][k] * m_kj * 2^e_dmin (columns j < 8)
  const h8 Bm0 = *reinterpret_cast<const h8 *>(&T.vm[n & 7][8 * g]);
  const h8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
  S.accm = mfma32(Am, n < 8 ? Bm0 : zero8, S.accm);
}

// Barrier of waves 0-3 only (the quantizing waves), through an LDS arrival counter, so
// that waves 4-7 need not wait for the quantization. Every waiting wave is in this
// workgroup, hence resident, and reaches each barrier; the bound on the wait (about
// 0.1 s) only keeps a fault from hanging the GPU: a wave that gives up sets
// kStatusBarrierTimeout in the device status word, which pkv_device_status() reports.
struct QuantWavesBarrier {
  uint32_t *arrivals;
  uint32_t target;
  unsigned *status;
  __device__ __forceinline__ void operator()() {
    target += 4;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if ((threadIdx.x & 63) == 0)
      __hip_atomic_fetch_add(arrivals, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    bool done = false;
    for (int spin = 0; spin < (1 << 22); ++spin) {
      if (__hip_atomic_load(arrivals, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) {
        done = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (!done && (threadIdx.x & 63) == 0)
      __hip_atomic_fetch_or(status, kStatusBarrierTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  }
};

// (kPrep) Stage a wave's preparation constants into LDS by the q rows' DMA path, so that
// the wait for q covers them and the compiler sees no load of its own to wait for (its
// waits cannot tell these loads from the block stages issued after them): the q_norm
// alphas (1 KB) into the wave's table area, the rope row's cos and sin (n_rot / 2 = 32
// floats each, zero-filled to 64 by the buffer range) into the q stage's tail.
__device__ __forceinline__ void issue_prep_consts(void *alpha_lds, void *tail_lds, u4s ra,
                                                  u4s rc, u4s rs, uint32_t lane) {
  const uint32_t da = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)((PKV_LDS void *)alpha_lds));
  const uint32_t dt = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)((PKV_LDS void *)tail_lds));
  uint32_t saved;
  asm volatile(
      "s_nop 4\n\t"  // VALU-written SGPRs (v_readfirstlane) read by VMEM: 5 wait states
      "s_mov_b32 %[sv], m0\n\t"
      "s_mov_b32 m0, %[da]\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o16], %[ra], 0 offen lds\n\t"
      "s_mov_b32 m0, %[dt]\n\ts_nop 0\n\t"
      "buffer_load_dword %[o4], %[rc], 0 offen lds\n\t"
      "s_add_u32 m0, %[dt], 0x100\n\ts_nop 0\n\t"
      "buffer_load_dword %[o4], %[rs], 0 offen lds\n\t"
      "s_mov_b32 m0, %[sv]"
      : [sv] "=&s"(saved)
      : [da] "s"(da), [dt] "s"(dt), [o16] "v"(16u * lane), [o4] "v"(4u * lane), [ra] "s"(ra),
        [rc] "s"(rc), [rs] "s"(rs)
      : "memory", "scc");
}

// The leading scalar arguments repeat what a workgroup needs before its first loads
// (segment 0's rows and key count for a one-segment launch, q, the fused region's words,
// k_new, the row strides rs_t | rs_h << 24, nwg): the build preloads them into SGPRs,
// so those loads wait for no kernel-argument fetch.
template <bool kPrep, int kSegs>
__global__ __launch_bounds__(kThreads) void q4k_decode_kernel(
    const uint8_t *k_0, const uint8_t *v_0, const float *q_0, uint32_t *words_0,
    const float *knew_0, uint64_t strides, int seq_k0, int nwg_0, DecodeArgsT<kSegs> a) {
  __shared__ Smem sm;
  constexpr bool kOne = kSegs == 1;
  if constexpr (kOne) {
    if ((int)blockIdx.x >= nwg_0 + kQuantFront(true, knew_0 != nullptr, nwg_0)) {
      // a combiner workgroup (in-launch combine)
      const TailArgs t{a.nwg, a.words, a.part, a.ml, a.q, a.q_out,
                       a.k_new != nullptr ? a.dq : nullptr, a.out, a.sl2, a.status};
      tail_combine<kPrep>(t, (int)blockIdx.x - a.nwg, &sm);
      return;
    }
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // the launch parity of an in-launch combine (0 otherwise), in the lowest bit of every
  // partial word this workgroup writes
  // (a one-segment launch has its words exactly when it combines in-launch). The word is
  // read without a branch (an empty buffer range reads 0) and the parity is formed where
  // it is stored, so the load is waited for at the first store, not here.
  uint32_t par_raw = 0u, par_on = 0u;
  if constexpr (kSegs == 1) {
    par_on = words_0 != nullptr ? 1u : 0u;
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc(words_0, 0, par_on ? 4 * Workspace::kFusedWords : 0, 0x00020000);
    par_raw = __builtin_amdgcn_raw_buffer_load_b32(rw, 4 * kWordGen, 0, kSC1);
  }
  const auto parity = [&]() { return (par_raw ^ par_on) & par_on; };
  const int kv = wave & 1, wsub = wave >> 1;
  // A one-row fused launch over fewer workgroups than CUs puts 4 workgroups in front that
  // only quantize the new rows (qx; the host sizes the grid by the same rule), so that no
  // decode workgroup's blocks wait behind the quantization.
  const int qx = kQuantFront(kOne, knew_0 != nullptr, nwg_0);
  const int wg = (int)blockIdx.x - qx;
  const int qwg = qx > 0 ? (int)blockIdx.x : wg;  // the first new row this workgroup quantizes
  const int n = lane & 15, g = lane >> 4;
  const int kvu = __builtin_amdgcn_readfirstlane(kv);
  const uint32_t rs_t = (uint32_t)(strides & 0xFFFFFFu);
  const int64_t rs_h = (int64_t)(strides >> 24);
  const LoadPlan P = make_plan(lane, rs_t);
  const uint32_t bstep = 4u * kBlk * rs_t;  // byte distance between a wave's blocks
  // LDS byte addresses of this wave's two stages
  const uint32_t st_lds0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(size_t)((PKV_LDS void *)&sm.run.st[wave][0]));

  // ---- pieces of this workgroup (wave-uniform): the blocks of [V0, V1) on the launch's
  // virtual block line, one piece per segment met (its blocks [pb0, pb1)), each with its
  // partial in slot wg + (the segment's index), distinct for every piece and
  // consecutive for the pieces of one segment.
  // (one segment: its blocks, or one virtual block for an empty one, split over nwg)
  const int nblk0 = (int)((seq_k0 + kBlk - 1) / kBlk);
  const int vq = kOne ? (nblk0 > 0 ? nblk0 : 1) / nwg_0 : a.vq;
  const int vr = kOne ? (nblk0 > 0 ? nblk0 : 1) % nwg_0 : a.vr;
  const int V0 = wg * vq + (wg < vr ? wg : vr);
  const int V1 = V0 + vq + (wg < vr ? 1 : 0);
  int ps = -1, pb0 = 0, pb1 = 0, slot = wg;
  DecodeSeg sgv = {};  // read only while a piece is held
  // paged device-list mode: (pi, pj) is the next segment the scan looks at
  int pi = 0, pj = 0;
  auto next_piece = [&]() -> bool {
    if constexpr (kSegs == 0) {
      if (ps < 0) {  // the first segment that may meet [V0, V1): found by arithmetic
        ps = 0;
        while (pi + 1 < a.nseg && a.pq[pi + 1].vstart <= V0) ++pi;
        const int rel = V0 - a.pq[pi].vstart;
        pj = rel > 0 ? rel / a.pstride : 0;
        if (pj >= a.pq[pi].npg) pj = a.pq[pi].npg - 1;
      }
      while (pi < a.nseg) {
        const PagedSeqArg &sq = a.pq[pi];
        const int64_t t0 = (int64_t)pj << a.page_lg, rest = sq.len - t0;
        const int64_t keys = rest < ((int64_t)1 << a.page_lg) ? rest : ((int64_t)1 << a.page_lg);
        const int nb = (int)((keys + kBlk - 1) / kBlk);
        const int vs = sq.vstart + pj * a.pstride;
        if (vs >= V1) return false;
        const int ve = vs + (nb > 0 ? nb : 1);
        const int k = sq.kfirst + pj, i = pi, j = pj;
        if (++pj >= sq.npg) {
          ++pi;
          pj = 0;
        }
        if (ve > V0) {
          const int64_t pg = sq.pages[j];
          sgv.k = a.kplane + pg * a.page_bytes;
          sgv.v = a.vplane + pg * a.page_bytes;
          sgv.seq_k = keys;
          sgv.t_new = 0;
          sgv.nblk = nb;
          sgv.wg0 = -1;
          sgv.qi = i;
          sgv.voff = vs;
          pb0 = (V0 > vs ? V0 : vs) - vs;
          const int e = (V1 < ve ? V1 : ve) - vs;
          pb1 = e < nb ? e : nb;
          slot = wg + k;
          return true;
        }
      }
      return false;
    } else {
    if constexpr (kSegs == 1) {  // one segment at voff 0: the range is the piece
      if (ps >= 0) return false;
      ps = 0;
      sgv.k = const_cast<uint8_t *>(k_0);
      sgv.v = const_cast<uint8_t *>(v_0);
      sgv.seq_k = seq_k0;
      sgv.t_new = a.seg[0].t_new;
      sgv.nblk = nblk0;
      sgv.wg0 = 0;
      sgv.qi = 0;
      sgv.voff = 0;
      pb0 = V0;
      pb1 = V1 < sgv.nblk ? V1 : sgv.nblk;
      return V0 < (sgv.nblk > 0 ? sgv.nblk : 1);
    }
    for (int s = ps + 1; s < a.nseg; ++s) {
      const int vs = a.seg[s].voff;
      if (vs >= V1) return false;
      const int nb = a.seg[s].nblk;
      const int ve = vs + (nb > 0 ? nb : 1);  // an empty segment holds one virtual block
      if (ve > V0) {
        ps = s;
        sgv = a.seg[s];
        pb0 = (V0 > vs ? V0 : vs) - vs;
        const int e = (V1 < ve ? V1 : ve) - vs;
        pb1 = e < nb ? e : nb;
        slot = wg + s;
        return true;
      }
    }
    return false;
    }
  };
  bool have = wg >= 0 && next_piece();
  if constexpr (kSegs == 0) {
    // The partial slots a workgroup owns run from wg + (segments ending at or before V0)
    // to wg + (segments starting before V1); its pieces fill them, except the last one
    // when its range does not end inside a segment: that slot gets an empty partial, so
    // that every slot in an output row's range holds one. The last segment starting
    // before V1 is (mi, mj).
    int mi = 0;
    while (mi + 1 < a.nseg && a.pq[mi + 1].vstart < V1) ++mi;
    const PagedSeqArg &sq = a.pq[mi];
    int mj = (V1 - 1 - sq.vstart) / a.pstride;
    if (mj >= sq.npg) mj = sq.npg - 1;
    const int64_t rest = sq.len - ((int64_t)mj << a.page_lg);
    const int64_t keys = rest < ((int64_t)1 << a.page_lg) ? rest : ((int64_t)1 << a.page_lg);
    const int nb = (int)((keys + kBlk - 1) / kBlk);
    if (sq.vstart + mj * a.pstride + (nb > 0 ? nb : 1) <= V1) {
      const int ms = wg + sq.kfirst + mj + 1;
      static_assert(kThreads * 8 == 16 * kPartRow, "one partial: 8 floats per thread");
      float *pz = a.part + ((int64_t)ms * 16 * kPartRow + 8 * tid);
      const f4 z = {0.f, 0.f, 0.f, 0.f};
      __builtin_nontemporal_store(z, reinterpret_cast<f4 *>(pz));
      __builtin_nontemporal_store(z, reinterpret_cast<f4 *>(pz) + 1);
      if (tid < 16) {
        float *mlo = reinterpret_cast<float *>(a.ml + (ms * 16 + tid));
        __builtin_nontemporal_store(-INFINITY, mlo);
        __builtin_nontemporal_store(0.0f, mlo + 1);
      }
    }
  }

  // Fused append: threads 0-255 (waves 0-3) of workgroup r quantize new row r (row
  // 4s + 2p + kv: segment s, K (p = 0) or V (p = 1), KV head kv; further rows go
  // round-robin when the grid is smaller) and publish it dequantized for the combine
  // step, which attends to the new key. The row is read before any staging load.
  // One output row (kOne): the quantization (about 3.5 us, a latency chain) runs first,
  // while the first blocks stream in (the row is waited for here, so that the compiler's
  // wait for it does not wait for a stage too), and the combiners have the new key's rows
  // early. Batched launches quantize after their block loops (kQuantLate): there the
  // rows go to a separate combine kernel, and a quantizing workgroup whose blocks start
  // late ends last (measured: config 5 1098.5 -> 1093.3 us/step, config 3 294 -> 311).
  constexpr bool kQuantLate = !kOne;
  const bool quant = knew_0 != nullptr && (qx > 0 ? wg < 0 : wg < 4 * (kOne ? 1 : a.nnew)) && tid < 256;
  float xq = 0.0f;
  PrepElem kpe[1] = {PrepElem{1.0f, 1.0f, 0.0f}};
  auto k_prep_elem = [&](int rs) {
    const int half = a.prep.n_rot >> 1;
    int64_t pos = 0;
    if constexpr (kSegs != 0) pos = a.seg[rs].t_new;
    return load_prep_elem(a.prep.k_alpha, a.prep.cos_tab + pos * half,
                          a.prep.sin_tab + pos * half, tid, 256, a.prep.n_rot);
  };
  // (kPrep, quantizing first) the quantizing waves, whose table areas hold the quantizer's
  // scratch until it is done, load the q preparation constants (q_norm alphas 4 lane ..
  // 4 lane + 3 and one rope cos / sin entry) with the new row and stage them in LDS after
  // quantizing; every other wave stages them by DMA below
  f4 qa4 = {1.0f, 1.0f, 1.0f, 1.0f};
  float rcos = 1.0f, rsin = 0.0f;
  if (quant) {
    const int p = (qwg >> 1) & 1, kvr = qwg & 1;
    xq = (p ? a.v_new : knew_0)[((int64_t)(qwg >> 2) * 2 + kvr) * 256 + tid];
    if constexpr (kPrep) {
      if (p == 0) kpe[0] = k_prep_elem(qwg >> 2);
      if constexpr (!kQuantLate) {
        qa4 = reinterpret_cast<const f4 *>(a.prep.q_alpha)[lane];
        const int half = a.prep.n_rot >> 1;
        if (have) {  // the first piece's q position (a workgroup without blocks has none)
          rcos = a.prep.cos_tab[sgv.t_new * half + (lane & (half - 1))];
          rsin = a.prep.sin_tab[sgv.t_new * half + (lane & (half - 1))];
        }
        asm volatile("" : "+v"(xq), "+v"(kpe[0].alpha), "+v"(kpe[0].c), "+v"(kpe[0].s),
                     "+v"(rcos), "+v"(rsin), "+v"(qa4));
      }
    } else if constexpr (!kQuantLate) {
      asm volatile("" : "+v"(xq));
    }
  }
  uint32_t *const qarrive = reinterpret_cast<uint32_t *>(&sm.run.t.tab[1].kd[0]);
  if (tid == 0) *qarrive = 0u;
  // Fused append (waves 0-3 of the quantizing workgroups, once): the rows, as above.
  auto quantize_rows = [&]() {
    // the quantization delays this workgroup's blocks or its partial: it outranks the
    // block loops of the waves sharing its SIMDs
    __builtin_amdgcn_s_setprio(3);
    QuantWavesBarrier bar{qarrive, 0u, a.status};
    if constexpr (kQuantLate) bar();  // all four are done with their tables (the scratch)
    for (int row = qwg; row < 4 * a.nnew; row += a.nwg) {
      const int rs = row >> 2, p = (row >> 1) & 1, kvr = row & 1;
      if (row != qwg) xq = (p ? a.v_new : a.k_new)[((int64_t)rs * 2 + kvr) * 256 + tid];
      uint8_t *dst;
      if constexpr (kSegs == 0) {  // row len of the page that holds token len
        const PagedSeqArg &sq = a.pq[rs];
        const int64_t pg = sq.pages[sq.len >> a.page_lg];
        dst = (p ? a.vplane : a.kplane) + pg * a.page_bytes +
              (sq.len & (((int64_t)1 << a.page_lg) - 1)) * rs_t + kvr * rs_h;
      } else {
        const DecodeSeg &rg = a.seg[rs];
        dst = (p ? rg.v : rg.k) + rg.t_new * rs_t + kvr * rs_h;
      }
      if constexpr (kPrep) {
        if (p == 0) {  // k_norm and rope of the new K row (bit-exact), then its quantization
          if (row != qwg) kpe[0] = k_prep_elem(rs);
          float xx[1] = {xq};
          prep_row<1>(xx, kpe, 256, a.prep.eps, a.prep.n_rot, sm.run.t.quant.prow,
                      &sm.run.t.quant.pm, tid, bar);
          xq = xx[0];
        }
      }
      float deq;
      q4k_quantize_superblock_lanes(xq, dst, &sm.run.t.quant.scr, tid, &deq, bar);
      bar.target += 12;  // the three barriers of that call
      store_sc1(a.dq + (int64_t)row * 256 + tid, deq);  // read by combiners on other XCDs
      if (a.ncomb > 0) {  // the row's word once all 256 values are stored
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        bar();
        if (tid == 0) store_sc1(a.words + kWordRow + row, parity());
      }
    }
    __builtin_amdgcn_s_setprio(0);
  };
  // One pass per piece; the fused append runs in the first. A workgroup without blocks
  // on its part of the line (have false) only quantizes, if it is a quantizing one.
  for (int pc = 0;; ++pc) {
    const bool qnow = quant && pc == 0;
    const DecodeSeg &sg = sgv;
    // ---- blocks of this wave: pb0 + wsub, pb0 + wsub + 4, ... below pb1
    // wave-uniform: loop control and the key mask stay scalar
    const int first = __builtin_amdgcn_readfirstlane(pb0 + wsub);
    const int nmine =
        __builtin_amdgcn_readfirstlane(have && first < pb1 ? (pb1 - first + 3) / 4 : 0);
    const uint8_t *kbase = sg.k + kvu * rs_h;
    const uint8_t *vbase = sg.v + kvu * rs_h;
    const int64_t seq_k = sg.seq_k;
    // rows of keys [0, seq_k) of this head; loads past them return zeros (masked keys)
    const uint32_t span = seq_k > 0 ? (uint32_t)(seq_k - 1) * rs_t + 144u : 0u;
    const u4s rk = make_rsrc(kbase, span), rv = make_rsrc(vbase, span);
    uint32_t boff = __builtin_amdgcn_readfirstlane((uint32_t)first * kBlk * rs_t);

    // ---- this wave's q rows, then its first block, into LDS. Every wave's q loads go out
    // before any stage load (one barrier), so q returns ahead of the block data.
    if (have) {
      if constexpr (kPrep) {
        if (kQuantLate || !qnow) {
          const int half = a.prep.n_rot >> 1;
          const int64_t ro = sg.t_new * half;
          issue_prep_consts(&sm.run.t.tab[wave].vc[0][0],
                            reinterpret_cast<uint8_t *>(&sm.run.st[wave][1]) + 8 * kQRow,
                            make_rsrc(a.prep.q_alpha, 1024u),
                            make_rsrc(a.prep.cos_tab + ro, (uint32_t)half * 4u),
                            make_rsrc(a.prep.sin_tab + ro, (uint32_t)half * 4u), (uint32_t)lane);
        }
      }
      const u4s rq = make_rsrc(q_0 + ((int64_t)sg.qi * 16 + 8 * kvu) * 256, 8 * 256 * 4);
      issue_q(&sm.run.st[wave][1], rq, 16u * lane);
    }
    __syncthreads();
    // every issued block has its first key below seq_k, so its offset is inside the range
    if (nmine > 0) issue_stage_at(st_lds0, P, rsrc_advance(rk, boff), rsrc_advance(rv, boff));

    // QK B operands: lane (n, g) takes q of head n % 8, elements 64g + 32(s/4) + 8(s%4) +
    // perm[slot], as the fp16 hi part (n < 8) or the lo remainder (n >= 8); S2 B operand:
    // the sums of sub-blocks 2g and 2g+1 (elements 64g..64g+31, 64g+32..64g+63, in order).
    // Built from the wave's own copy of q, so no workgroup barrier is needed.
    h8 qb[8];
    h4 q2 = {0, 0, 0, 0};
    auto build_q = [&]() {
      // q was issued before this wave's stage loads (12): once at most 12 loads are
      // outstanding, q has landed
      if (nmine > 0)
        asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      if constexpr (kPrep && !kQuantLate) {
        if (qnow) {  // after quantizing: the constants into this wave's vc / vm and tail
          float *tail = reinterpret_cast<float *>(&sm.run.st[wave][1]) + 8 * (kQRow / 4);
          reinterpret_cast<f4 *>(&sm.run.t.tab[wave].vc[0][0])[lane] = qa4;
          tail[lane] = lane < 32 ? rcos : 0.0f;
          tail[64 + lane] = lane < 32 ? rsin : 0.0f;
          __builtin_amdgcn_wave_barrier();
        }
      }
      const float *qrow = reinterpret_cast<const float *>(&sm.run.st[wave][1]) + (n & 7) * (kQRow / 4) + 64 * g;
      constexpr int perm[8] = {0, 2, 1, 3, 4, 6, 5, 7};
      float qsum[2] = {0.0f, 0.0f};
      // hi lanes (n < 8) take fp16(q), lo lanes fp16(q - fp16(q)): both are fp16(q - c)
      // with c = fp16(q) masked to zero on the hi lanes
      const uint32_t lo_mask = n < 8 ? 0u : 0xFFFFFFFFu;
      auto convert = [&](int st, const float (&v8)[8]) {
#pragma unroll
        for (int k = 0; k < 8; ++k) qsum[st >> 2] += v8[k];
        uint32_t w[4];
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
          const float a0 = v8[perm[2 * pp]], a1 = v8[perm[2 * pp + 1]];
          const h2 h = {(_Float16)a0, (_Float16)a1};
          const uint32_t c = as_u(h) & lo_mask;
          w[pp] = fp16_sub2(a0, a1, c);
        }
        qb[st] = __builtin_bit_cast(h8, u4{w[0], w[1], w[2], w[3]});
      };
      if constexpr (kPrep) {
        // q_norm and rope in registers: v[st][k] is element 8 st + k of the lane's 64
        // (64 g ..) of row n % 8; the row's 4 lanes (g = 0..3) pool their sums of squares,
        // and the g = 0 lanes hold every rope pair (j, j + 32) of n_rot = 64. q feeds the
        // attention only: sums in any order and x * (1 / m) are within its tolerance.
        float v[8][8];
#pragma unroll
        for (int st = 0; st < 8; ++st) {
          const float4 r0 = *reinterpret_cast<const float4 *>(qrow + 8 * st);
          const float4 r1 = *reinterpret_cast<const float4 *>(qrow + 8 * st + 4);
          v[st][0] = r0.x; v[st][1] = r0.y; v[st][2] = r0.z; v[st][3] = r0.w;
          v[st][4] = r1.x; v[st][5] = r1.y; v[st][6] = r1.z; v[st][7] = r1.w;
        }
        float ss = 0.0f;
#pragma unroll
        for (int st = 0; st < 8; ++st)
#pragma unroll
          for (int k = 0; k < 8; ++k) ss = fmaf(v[st][k], v[st][k], ss);
        {
          const uint32_t u = __builtin_bit_cast(uint32_t, ss);
          const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
          const uint32_t r0 = r[0], r1 = r[1];
          ss = __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
        }
        {
          const uint32_t u = __builtin_bit_cast(uint32_t, ss);
          const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
          const uint32_t r0 = r[0], r1 = r[1];
          ss = __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
        }
        const float inv = 1.0f / __builtin_sqrtf(ss * (1.0f / 256.0f) + a.prep.eps);
        const float *al = reinterpret_cast<const float *>(&sm.run.t.tab[wave].vc[0][0]) + 64 * g;
#pragma unroll
        for (int st = 0; st < 8; ++st) {
          const float4 a0 = *reinterpret_cast<const float4 *>(al + 8 * st);
          const float4 a1 = *reinterpret_cast<const float4 *>(al + 8 * st + 4);
          const float a8[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
          for (int k = 0; k < 8; ++k) v[st][k] = v[st][k] * inv * a8[k];
        }
        if (g == 0) {
          const float *tail = reinterpret_cast<const float *>(&sm.run.st[wave][1]) + 8 * (kQRow / 4);
#pragma unroll
          for (int st = 0; st < 4; ++st) {
            const float4 c0 = *reinterpret_cast<const float4 *>(tail + 8 * st);
            const float4 c1 = *reinterpret_cast<const float4 *>(tail + 8 * st + 4);
            const float4 s0 = *reinterpret_cast<const float4 *>(tail + 64 + 8 * st);
            const float4 s1 = *reinterpret_cast<const float4 *>(tail + 64 + 8 * st + 4);
            const float c8[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
            const float s8[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
            for (int k = 0; k < 8; ++k) {
              const float x1 = v[st][k], x2 = v[st + 4][k];
              v[st][k] = x1 * c8[k] - x2 * s8[k];
              v[st + 4][k] = x1 * s8[k] + x2 * c8[k];
            }
          }
        }
        if (wg == sg.wg0 && wsub == 0 && n < 8) {  // the combine's copy of the prepared q
          float *qo = a.q_out + ((int64_t)sg.qi * 16 + 8 * kvu + n) * 256 + 64 * g;
          if (a.ncomb > 0) {  // read by combiners of this launch, on other XCDs
#pragma unroll
            for (int st = 0; st < 8; ++st)
#pragma unroll
              for (int k = 0; k < 8; ++k) store_sc1(qo + 8 * st + k, v[st][k]);
            // (the wave's word follows below, once every lane's stores are done)
          } else {
#pragma unroll
            for (int st = 0; st < 8; ++st) {
              *reinterpret_cast<float4 *>(qo + 8 * st) = float4{v[st][0], v[st][1], v[st][2], v[st][3]};
              *reinterpret_cast<float4 *>(qo + 8 * st + 4) = float4{v[st][4], v[st][5], v[st][6], v[st][7]};
            }
          }
        }
        if (a.ncomb > 0 && wg == sg.wg0 && wsub == 0) {  // this wave's q rows are stored
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
          if (lane == 0) store_sc1(a.words + kWordQ + kvu, parity());
        }
#pragma unroll
        for (int st = 0; st < 8; ++st) convert(st, v[st]);
      } else {
#pragma unroll
        for (int st = 0; st < 8; ++st) {
          const float4 r0 = *reinterpret_cast<const float4 *>(qrow + 32 * (st >> 2) + 8 * (st & 3));
          const float4 r1 = *reinterpret_cast<const float4 *>(qrow + 32 * (st >> 2) + 8 * (st & 3) + 4);
          const float v8[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
          convert(st, v8);
        }
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const _Float16 hi = (_Float16)qsum[t];
        q2[t] = (n < 8) ? hi : (_Float16)(qsum[t] - (float)hi);
      }
    };
    static_assert(kLoadsPerStage == 12, "the vmcnt above counts one stage of loads");

    if (qnow && (!kQuantLate || !have)) quantize_rows();
    if (!have) {
      if constexpr (kSegs == 1) {
        // (the one-segment plan gives every workgroup a block; should it not, its slot
        // holds an empty partial for the combiners)
        if (a.ncomb > 0) {
          float *pz = a.part + ((int64_t)slot * 16 * kPartRow + 8 * tid);
#pragma unroll
          for (int x = 0; x < 8; ++x) store_sc1(pz + x, tag_par(0.0f, parity()));
          if (tid < 16) {
            float *mlo = reinterpret_cast<float *>(a.ml + (slot * 16 + tid));
            store_sc1(mlo, tag_par(-INFINITY, parity()));
            store_sc1(mlo + 1, tag_par(0.0f, parity()));
          }
        }
      }
      return;
    }
    build_q();

    WaveState S;
#pragma unroll
    for (int T2 = 0; T2 < 16; ++T2) S.acc[T2] = f4{0.f, 0.f, 0.f, 0.f};
    S.accm = f4{0.f, 0.f, 0.f, 0.f};
    S.m_run = -INFINITY;
    S.lsum = 0.0f;
    WaveTab &T = sm.run.t.tab[wave];
    if (nmine > 0) {
      const Masks MK = {vconst(0x000F000Fu), vconst(0x00F000F0u), vconst(0x64006400u)};
      const KScaleSel ks = make_kscale_sel(g);
      const float clamp_raw = kClampL2 / a.sl2, lazy_raw = kLazy / a.sl2;
      const VScaleSel vs = make_vscale_sel(lane);
      for (int i = 0; i < nmine; ++i) {
        const int si = i & 1;  // block i uses stage i % 2
        // The two waves of a SIMD are issued oldest-first at equal priority, which lets
        // the older one run ahead and leaves the younger to finish alone. Lowering the
        // priority with each block done keeps the one behind first in line.
        if (i == 0)
          __builtin_amdgcn_s_setprio(2);
        else if (i == 1)
          __builtin_amdgcn_s_setprio(1);
        else if (i == 2)
          __builtin_amdgcn_s_setprio(0);
        if (i + 1 < nmine) {  // block i+1 streams in while block i is processed
          issue_stage_at(st_lds0 + (uint32_t)(1 - si) * (uint32_t)sizeof(Stage), P,
                         rsrc_advance(rk, boff + bstep), rsrc_advance(rv, boff + bstep));
          asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
        } else {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        const Stage &st = sm.run.st[wave][si];
        BlockWords W;
        load_block_words(st, lane, W);
        __builtin_amdgcn_sched_barrier(0);  // keep the K reads ahead of their phases
        QKOut qo;
        float pv[8];
        phase_q(W, qb, q2, MK, ks, qo);
        phase_s(W, qo, S, (int)(seq_k - (int64_t)(first + 4 * i) * kBlk), a.sl2, clamp_raw,
                lazy_raw, lane, pv);
        phase_p(st, W, S, T, pv, MK, vs, lane);
        // every LDS read of this stage has completed before it is refilled
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        boff += bstep;
      }
      __builtin_amdgcn_s_setprio(0);
    }
    if (kQuantLate && qnow) quantize_rows();
    // ---- epilogue: per-wave reductions, then the four waves of each KV head merged into
    // this workgroup's partial
    S.lsum += __shfl_xor(S.lsum, 16);
    S.lsum += __shfl_xor(S.lsum, 32);
    // Row halves: the hi rows 0-7 sit in lanes g < 2 and the lo rows 8-15 of the same
    // heads 32 lanes up. One v_permlane32_swap sums them for two tiles at once: afterwards
    // lanes 0-31 hold tile T2 and lanes 32-63 tile T2 + 8, both for rows (heads)
    // 4 (g & 1) + i.
    const int gr = g & 1, gh = g >> 1;
    f4 hs[8];
#pragma unroll
    for (int T2 = 0; T2 < 8; ++T2)
#pragma unroll
      for (int i = 0; i < 4; ++i) hs[T2][i] = pair_sum32(S.acc[T2][i], S.acc[T2 + 8][i]);
    // min term, paired alike: cm0 is row 4 (g & 1) + g / 2, cm1 row 4 (g & 1) + 2 + g / 2
    // (column j = n)
    const float cm0 = pair_sum32(S.accm[0], S.accm[1]), cm1 = pair_sum32(S.accm[2], S.accm[3]);
    // Exchange through this wave's own table area: ml = {m of heads 0-7 (log2 units), l,
    // f * l}, read by the other waves after the barrier; then cmin[head][j] * f.
    float(*cmin)[8] = reinterpret_cast<float(*)[8]>(&T.kd[0]);
    float *ml = T.vmd;
    if (g == 0 && n < 8) {
      ml[n] = S.m_run * a.sl2;
      ml[8 + n] = S.lsum;
    }
    __syncthreads();  // every wave has left the loop: the stage buffers become the merge area
    // weights f = 2^(m - M) of this wave's rows against the four waves of its KV head
    auto weight = [&](int h) {
      float M = -INFINITY;
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) M = fmaxf(M, sm.run.t.tab[2 * s4 + kv].vmd[h]);
      const float mine = ml[h];
      return (mine == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mine - M);
    };
    float fr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) fr[i] = weight(4 * gr + i);
    // cmin * f, written and read back by this wave only (its LDS operations stay in order)
    if (n < 8) {
      cmin[4 * gr + gh][n] = cm0 * (gh ? fr[1] : fr[0]);
      cmin[4 * gr + 2 + gh][n] = cm1 * (gh ? fr[3] : fr[2]);
    }
    // scaled output rows: acc * f - cmin[row][e / 32] * f, one float4 per tile
#pragma unroll
    for (int T2 = 0; T2 < 8; ++T2) {
      const int Tt = T2 + 8 * gh;
      const int j = tile_e(Tt, n) >> 5;
      float4 v;
      v.x = fmaf(hs[T2][0], fr[0], -cmin[4 * gr + 0][j]);
      v.y = fmaf(hs[T2][1], fr[1], -cmin[4 * gr + 1][j]);
      v.z = fmaf(hs[T2][2], fr[2], -cmin[4 * gr + 2][j]);
      v.w = fmaf(hs[T2][3], fr[3], -cmin[4 * gr + 3][j]);
      sm.merge.o[wave][Tt][gr][n] = v;
    }
    if (g == 0 && n < 8) ml[16 + n] = weight(n) * ml[8 + n];
    __syncthreads();
    // ---- merge: item (kv, T2, g2, n) sums rows 4 g2 .. 4 g2 + 3 of KV head kv over its four
    // waves and stores them at tile-order entry 16 T2 + n of heads 8 kv + 4 g2 + i
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int item = tid + kThreads * it;
      const int n2 = item & 15, g2 = (item >> 4) & 1, T2 = (item >> 5) & 15, kv2 = item >> 9;
      float4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const float4 v = sm.merge.o[2 * s4 + kv2][T2][g2][n2];
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
      }
      // one 32-bit index (slot < 2^16), so that no per-lane address outlives the piece
      float *d0 = a.part + ((slot * 16 + 8 * kv2 + 4 * g2) * kPartRow + 16 * T2 + n2);
      // lowest bit: the launch parity (in-launch combine) or zero
      if (a.ncomb > 0) {
        store_sc1(d0, tag_par(acc.x, parity()));
        store_sc1(d0 + kPartRow, tag_par(acc.y, parity()));
        store_sc1(d0 + 2 * kPartRow, tag_par(acc.z, parity()));
        store_sc1(d0 + 3 * kPartRow, tag_par(acc.w, parity()));
      } else {
        __builtin_nontemporal_store(untag(acc.x), d0);
        __builtin_nontemporal_store(untag(acc.y), d0 + kPartRow);
        __builtin_nontemporal_store(untag(acc.z), d0 + 2 * kPartRow);
        __builtin_nontemporal_store(untag(acc.w), d0 + 3 * kPartRow);
      }
    }
    if (tid < 16) {
      const int kv2 = tid >> 3, h = tid & 7;
      float M = -INFINITY, L = 0.0f;
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        M = fmaxf(M, sm.run.t.tab[2 * s4 + kv2].vmd[h]);
        L += sm.run.t.tab[2 * s4 + kv2].vmd[16 + h];
      }
      float *mlo = reinterpret_cast<float *>(a.ml + (slot * 16 + tid));
      if (a.ncomb > 0) {
        store_sc1(mlo, tag_par(M, parity()));
        store_sc1(mlo + 1, tag_par(L, parity()));
      } else {
        __builtin_nontemporal_store(untag(M), mlo);
        __builtin_nontemporal_store(untag(L), mlo + 1);
      }
    }
    if constexpr (kSegs == 1) break;  // one segment: one piece
    if (!next_piece()) break;
    // the next piece's q and blocks refill the stage buffers, the merge area until here
    __syncthreads();
  }
}


}  // namespace

// Plan and launch the decode and combine kernels over n <= kMaxSegs segments.
// kPrep: q_norm / k_norm / rope of the step's q and new k run inside the kernels (prep
// must then be set). Each translation unit instantiates one kPrep only, so that the
// instantiations are optimised separately.
template <bool kPrep>
static int launch_decode_segments(const DecodeSegIn *in, int n, const float *q,
                                  const float *k_new, const float *v_new, float *out,
                                  int64_t rs_t, int64_t rs_h, float scale, Workspace &ws,
                                  hipStream_t s, const DecodePrep *prep = nullptr) {
  if (!decode_head_stride_fits(rs_h)) return PKV_ERR_UNSUPPORTED;
  DecodeArgsT<kMaxSegs> d;
  const bool fused = k_new != nullptr;
  for (int i = 0; i < n; ++i) {
    d.seg[i].k = in[i].k;
    d.seg[i].v = in[i].v;
    d.seg[i].seq_k = fused ? in[i].seq_k - 1 : in[i].seq_k;  // the new key joins in the combine
    d.seg[i].t_new = in[i].seq_k - 1;
    d.seg[i].nblk = (int)((d.seg[i].seq_k + kBlk - 1) / kBlk);
    d.seg[i].qi = i;
  }
  d.nnew = n;
  // Stream-K plan: the segments' blocks on one virtual line (segment i from voff, an
  // empty segment as one block), with a gap of kPieceGap blocks before every segment
  // after the first, the estimated cost of one more pass (epilogue, q staging and the
  // first block's latency), so that a workgroup whose range crosses a boundary gets
  // fewer blocks. The nwg workgroups split the V blocks into ranges of vq or vq + 1
  // (about 4 blocks or more each, one per wave pair; at most one workgroup per CU),
  // the vr longer ones first. Workgroup w's piece of segment s writes partial slot
  // w + s; segment s has pieces on the workgroups from the one whose range holds its
  // first virtual block to the one that holds its last, so its slots are consecutive.
  int V = 0;
  for (int i = 0; i < n; ++i) {
    if (i > 0) V += kPieceGap;
    d.seg[i].voff = V;
    V += d.seg[i].nblk > 0 ? d.seg[i].nblk : 1;
  }
  int nwg = (V + 3) / 4;
  if (nwg > kMainWGs) nwg = kMainWGs;
  if (nwg < 1) nwg = 1;
  CombineArgs c;
  const int vq = V / nwg, vr = V % nwg;
  // the workgroup whose range holds virtual block x (ranges of vq + 1, vr times, then vq)
  auto wg_of = [&](int x) {
    const int big = vr * (vq + 1);
    return x < big ? x / (vq + 1) : vr + (x - big) / vq;
  };
  for (int i = 0; i < n; ++i) {
    const int vs = d.seg[i].voff, ve = vs + (d.seg[i].nblk > 0 ? d.seg[i].nblk : 1);
    const int w0 = wg_of(vs), w1 = wg_of(ve - 1);
    d.seg[i].wg0 = w0;
    c.wg0[i] = w0 + i;
    c.wg1[i] = w1 + i + 1;
  }
  const int wg = nwg + n - 1;  // partial slots
  d.nseg = n;
  d.nwg = nwg;
  d.vq = vq;
  d.vr = vr;
  d.rs_t = rs_t;
  d.rs_h = rs_h;
  d.sl2 = scale * kLog2e;
  d.q = q;
  d.k_new = k_new;
  d.v_new = v_new;
  const size_t part_floats = (size_t)wg * 16 * kPartRow, ml_floats = (size_t)wg * 16 * 2;
  const size_t need = (part_floats + ml_floats + (size_t)n * 4 * 256 +
                       (kPrep ? (size_t)n * 16 * 256 : 0)) *
                      sizeof(float);
  int rc = ws.reserve(need);
  if (rc) return rc;
  d.part = static_cast<float *>(ws.ptr);
  d.ml = reinterpret_cast<float2 *>(d.part + part_floats);
  d.dq = d.part + part_floats + ml_floats;
  d.q_out = d.dq + (size_t)n * 4 * 256;
  d.prep = kPrep ? *prep : DecodePrep{};
  rc = device_status_word(&d.status);
  if (rc) return rc;
  d.ncomb = 0;
  d.words = nullptr;
  d.out = out;
  // one output row over a full grid: the combine runs inside the decode launch, on the
  // workspace's fused region (every such launch writes all of its slots, which the
  // parity protocol needs); a no-alloc call has no fused region
  if (n == 1 && nwg == Workspace::kFusedSlots && decode_fuse_enabled() && !ws.fixed) {
    rc = ws.reserve_fused(s);
    if (rc) return rc;
    float *f = static_cast<float *>(ws.fused);
    d.ncomb = kTailWGs;
    d.part = f;
    d.ml = reinterpret_cast<float2 *>(f + (size_t)Workspace::kFusedSlots * 16 * kPartRow);
    d.words = reinterpret_cast<uint32_t *>(f + (size_t)Workspace::kFusedSlots * 16 * (kPartRow + 2));
  }
  if (n == 1) {
    DecodeArgsT<1> d1;
    static_cast<DecodeArgsBase &>(d1) = d;
    d1.seg[0] = d.seg[0];
    const int qx = kQuantFront(true, fused, nwg);
    hipLaunchKernelGGL((q4k_decode_kernel<kPrep, 1>), dim3((unsigned)(qx + nwg + d.ncomb)), dim3(kThreads),
                       0, s, d.seg[0].k, d.seg[0].v, q, d.words, k_new,
                       decode_strides(rs_t, rs_h), (int)d.seg[0].seq_k, nwg, d1);
    PKV_HIP(hipGetLastError());
    if (d.ncomb > 0) return PKV_OK;
  } else {
    hipLaunchKernelGGL((q4k_decode_kernel<kPrep, kMaxSegs>), dim3((unsigned)nwg), dim3(kThreads), 0,
                       s, d.seg[0].k, d.seg[0].v, q, d.words, k_new, decode_strides(rs_t, rs_h),
                       (int)d.seg[0].seq_k, nwg, d);
  }
  PKV_HIP(hipGetLastError());
  c.part = d.part;
  c.ml = d.ml;
  c.q = kPrep ? d.q_out : q;
  c.dq = fused ? d.dq : nullptr;
  c.out = out;
  c.sl2 = d.sl2;
  if (const int rc_ = launch_combine(c, n, s)) return rc_;
  return PKV_OK;
}

}  // namespace pkv
