// Gated output projection, batched form for many tokens (a prefill chunk, a large decode
// batch), gfx950 MFMA: the step after the attention (paramecia-model/src/qwen3_next.rs:
// 2657-2680), out[t][o] = sum_i W[o][i] * x[t][i] * sigmoid(g[t][i]), with W a GGUF Q4K,
// Q5K or Q6K attn_output (self.wo, models/with_tracing.rs:253-300). The per-token form
// (pkv_oproj.hip) re-reads and re-decodes every weight once per token; here each decoded
// weight feeds 32 tokens through v_mfma_f32_16x16x32_f16.
//
// Exactness of the fp16 operands:
//   - activations: a pre-pass gates each token row, scales it by a power of two so that
//     its largest magnitude lies in [2^14, 2^15) (exact), and splits every value into
//     hi = fp16(y) and lo = fp16(y - hi): hi + lo carries about 22 bits, so two MFMAs per
//     weight operand give near-f32 products. The pre-pass also writes each 32-input
//     sub-block's sum (scaled by 2^-6 so that it fits fp16, again as hi + lo) for the min
//     term, and 2^-e per token for the epilogue.
//   - Q4K/Q5K weights: code n (0..15 / 0..31) times its 6-bit sub-block scale sc is an
//     integer below 2048, exact in fp16: fma(1024 + n, sc, -1024 sc) with 1024 + n built
//     from the code bits by v_perm (fp16 0x6400 | n). The MFMA then sums sc * n * x over a
//     whole superblock, and the epilogue of each superblock adds d * that - dmin * (sum_j
//     m_j * xsum_j), the latter one v_mfma_f32_16x16x16_f16 over the 8 sub-blocks (hi and
//     lo sums in k 0-7 and 8-15).
//   - Q6K weights: (q - 32) * sc reaches 4096, not exact in fp16, so the int8 scale is
//     split as sc = 16 sh + sl (sl 0..15, sh -8..7): (q - 32) sl and 16 sh (q - 32) are
//     both exact, two B operands into the same accumulator, d applied per superblock.
//
// Work split: a workgroup of 4 waves owns 256 output rows (64 per wave: four 16-row MFMA
// tiles) and 32 tokens (two 16-token tiles), over a range of superblocks (split-K when the
// grid would otherwise leave CUs idle; a reduce kernel then sums the partials in split
// order). Per superblock, the tokens' fp16 fragments (32 KB) and the 256 rows' weight
// blocks are loaded into registers while the previous superblock computes, and stored to
// LDS between two barriers: the only waits for memory sit right before those stores, and
// each wave decodes its rows' B fragments from LDS. Tiles are placed on XCDs in compact
// groups (tile_of) so that an XCD's L2 serves both operands to several workgroups.
#include "pkv_mfma_common.hpp"

namespace pkv {
namespace {

enum : int { kMQ4K = 12, kMQ5K = 13, kMQ6K = 14 };
constexpr int kMxTargetWGs = 256;

// ---- pre-pass: gate, per-token power-of-two scale, fp16 hi/lo MFMA A fragments

struct XprepArgs {
  const float *attn, *gate;  // [T][K]; gate may be null
  int T, K;
  u4 *xh, *xl;  // [T_pad][K / 8]: fp16 hi and lo of the scaled gated inputs, 8 per unit
  h4 *xs;       // [T_pad][K / 256][4]: per superblock, the 8 sub-block sums' hi halves
                // then their lo halves (the min-term MFMA's k 0-7 and 8-15)
  float *inv;   // [T_pad] 2^-e
};

__device__ __forceinline__ float sigmoid_fast(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f));
}

// One workgroup per (padded) token; thread tid owns 8-input pieces tid + 256 p.
template <int kP>
__global__ __launch_bounds__(256) void oproj_xprep_kernel(XprepArgs a) {
#pragma clang fp contract(off)
  __shared__ float red[4];
  const int t = blockIdx.x, tid = threadIdx.x;
  const bool live = t < a.T;
  const int SB = a.K >> 8;
  float y[kP][8];
  float mx = 0.0f;
#pragma unroll
  for (int p = 0; p < kP; ++p) {
    const int e0 = 8 * (tid + 256 * p);
    float4 x[2] = {float4{0.f, 0.f, 0.f, 0.f}, float4{0.f, 0.f, 0.f, 0.f}};
    float4 g[2] = {float4{0.f, 0.f, 0.f, 0.f}, float4{0.f, 0.f, 0.f, 0.f}};
    if (live) {
      const float4 *xp = reinterpret_cast<const float4 *>(a.attn + (int64_t)t * a.K + e0);
      x[0] = xp[0];
      x[1] = xp[1];
      if (a.gate != nullptr) {
        const float4 *gp = reinterpret_cast<const float4 *>(a.gate + (int64_t)t * a.K + e0);
        g[0] = gp[0];
        g[1] = gp[1];
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float xv[4] = {x[h].x, x[h].y, x[h].z, x[h].w};
      const float gv[4] = {g[h].x, g[h].y, g[h].z, g[h].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = a.gate != nullptr ? xv[i] * sigmoid_fast(gv[i]) : xv[i];
        y[p][4 * h + i] = v;
        mx = fmaxf(mx, fabsf(v));
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int e = 0;
  if (mx > 0.0f && mx <= 3.4e38f) {
    int E;
    (void)frexpf(mx, &E);  // mx = f 2^E, f in [0.5, 1): mx 2^(15 - E) in [2^14, 2^15)
    e = 15 - E;
    e = e > 126 ? 126 : e;
  }
  if (tid == 0) a.inv[t] = live ? __builtin_ldexpf(1.0f, -e) : 0.0f;
#pragma unroll
  for (int p = 0; p < kP; ++p) {
    const int piece = tid + 256 * p, kb = piece >> 2, q = piece & 3;
    uint32_t hw[4], lw[4];
    float s8 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v0 = __builtin_ldexpf(y[p][2 * i], e), v1 = __builtin_ldexpf(y[p][2 * i + 1], e);
      const _Float16 h0 = (_Float16)v0, h1 = (_Float16)v1;
      const _Float16 l0 = (_Float16)(v0 - (float)h0), l1 = (_Float16)(v1 - (float)h1);
      hw[i] = (uint32_t)__builtin_bit_cast(uint16_t, h0) |
              ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
      lw[i] = (uint32_t)__builtin_bit_cast(uint16_t, l0) |
              ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
      s8 += v0 + v1;
    }
    a.xh[(int64_t)t * (a.K >> 3) + piece] = u4{hw[0], hw[1], hw[2], hw[3]};
    a.xl[(int64_t)t * (a.K >> 3) + piece] = u4{lw[0], lw[1], lw[2], lw[3]};
    // the sub-block's sum: pieces 4 kb .. 4 kb + 3 sit in threads 4 m .. 4 m + 3
    s8 += __shfl_xor(s8, 1);
    s8 += __shfl_xor(s8, 2);
    if (q == 0) {
      const float xsum = s8 * 0.015625f;  // 2^-6: |sum| < 2^20 becomes < 2^14
      const _Float16 xh = (_Float16)xsum, xl = (_Float16)(xsum - (float)xh);
      const int sb = kb >> 3, j = kb & 7;
      _Float16 *rec = reinterpret_cast<_Float16 *>(a.xs + ((int64_t)t * SB + sb) * 4);
      rec[j] = xh;
      rec[8 + j] = xl;
    }
  }
}

// ---- the workgroup's weights of one superblock, staged in LDS: row r of the 256 at
// Wr + r * kRowImg. Q4K / Q5K: the 144 / 176-byte block as stored. Q6K: the 53 dwords from
// the block's dword-aligned start (the block begins `sh` = 0 or 2 bytes in; its last byte
// at image offset 209 + sh), of which dword 52 is rebuilt from two 2-byte loads so that no
// load reaches past the block.

template <int kFmt>
struct WFmt {
  static constexpr int kBB = kFmt == kMQ4K ? 144 : kFmt == kMQ5K ? 176 : 210;
  static constexpr int kRowImg = kFmt == kMQ6K ? 224 : kBB;  // LDS bytes per row (16 B units)
  // 16-byte copy units per row (Q6K: dwords 0-51 of the image; dword 52 separately)
  static constexpr int kUnits = kFmt == kMQ6K ? 13 : kBB / 16;
  static constexpr int kPer = kUnits;  // units per thread (256 rows, 256 threads)
};

// One 16-byte copy unit u (row u / kUnits, piece u % kUnits) of superblock s.
template <int kFmt>
__device__ __forceinline__ u4 load_unit(const uint8_t *w, int64_t row_bytes, int row0, int N,
                                        int s, int u) {
  using F = WFmt<kFmt>;
  const int r = u / F::kUnits, k = u - r * F::kUnits;
  int n = row0 + r;
  n = n < N ? n : N - 1;
  const int64_t B = (int64_t)n * row_bytes + (int64_t)F::kBB * s;
  if constexpr (kFmt == kMQ6K) {
    // dwords 4 k .. 4 k + 3 of the image, from the block's dword-aligned start
    struct alignas(4) W4 { uint32_t v[4]; };
    const W4 q = *reinterpret_cast<const W4 *>(w + (B & ~(int64_t)3) + 16 * k);
    return u4{q.v[0], q.v[1], q.v[2], q.v[3]};
  } else {
    return *reinterpret_cast<const u4 *>(w + B + 16 * k);
  }
}

// N dwords of an LDS byte image from an even byte offset (aligned dwords shifted by
// v_alignbyte; reads one dword past the last byte)
// Q6K image dword 52 (image bytes 208-211) of row r: the block's last bytes 208 - sh ..
// 209 - sh, from two 2-byte loads (raw here, combined when stored) so that no load reaches
// past the block.
__device__ __forceinline__ void load_q6_tail(const uint8_t *w, int64_t row_bytes, int row0, int N,
                                             int s, int r, uint32_t &h0, uint32_t &h1) {
  int n = row0 + r;
  n = n < N ? n : N - 1;
  const int64_t B = (int64_t)n * row_bytes + 210 * (int64_t)s;
  h0 = *reinterpret_cast<const uint16_t *>(w + B + 206);
  h1 = *reinterpret_cast<const uint16_t *>(w + B + 208);
}

template <int N>
__device__ __forceinline__ void img_dwords(const uint8_t *img, int off, uint32_t (&o)[N]) {
  const uint32_t *p = reinterpret_cast<const uint32_t *>(img + (off & ~3));
  const uint32_t sh = off & 3;
  uint32_t d[N + 1];
#pragma unroll
  for (int i = 0; i <= N; ++i) d[i] = p[i];
#pragma unroll
  for (int i = 0; i < N; ++i) o[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], sh);
}

// {1024 + b0, 1024 + b1} and {1024 + b2, 1024 + b3} as fp16 pairs from the bytes of x
// (each below 64): v_perm selects byte 4 of the pair (src0 = 0x64646464) as every high byte.
__device__ __forceinline__ uint32_t magic_lo(uint32_t x) {
  return __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u);
}
__device__ __forceinline__ uint32_t magic_hi(uint32_t x) {
  return __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u);
}
__device__ __forceinline__ h2 h2_splat(float v) {
  const _Float16 h = (_Float16)v;
  return h2{h, h};
}
// 8 codes (bytes of x0, x1) scaled: fma(1024 + code, s, c) per half
__device__ __forceinline__ h8 scaled_codes(uint32_t x0, uint32_t x1, h2 s, h2 c) {
  const h2 p0 = pk_fma(as_h2(magic_lo(x0)), s, c), p1 = pk_fma(as_h2(magic_hi(x0)), s, c);
  const h2 p2 = pk_fma(as_h2(magic_lo(x1)), s, c), p3 = pk_fma(as_h2(magic_hi(x1)), s, c);
  return h8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

struct MxArgs {
  const u4 *xh, *xl;  // [T_pad][K / 8]
  const h4 *xs;       // [T_pad][K / 256][4]
  const float *inv;
  const uint8_t *w;
  int64_t row_bytes;
  float *part;  // [S][T][N] (S > 1)
  float *out;   // [T][N] (S == 1)
  int T, N, KB, SB, sb_per_split, S;
  int rbs, tbs;  // row blocks, token blocks
};

// Tile (split, row block, token block) of workgroup `id`. Workgroups are dealt to the 8
// XCDs in turn (id % 8), and each XCD has its own L2: when the grid divides by 8, XCD x
// takes tiles x C .. x C + C - 1 (C = grid / 8) of an order in which consecutive tiles
// form compact blocks, up to 4 row blocks by C / 4 token blocks, so that an XCD's
// workgroups share both their weights and their token fragments in its L2.
__device__ __forceinline__ void tile_of(const MxArgs &a, int id, int G, int &split, int &rb,
                                        int &tbk) {
  const int tile = (G & 7) == 0 ? (id & 7) * (G >> 3) + (id >> 3) : id;
  const int per_split = a.rbs * a.tbs;
  split = tile / per_split;
  const int rem = tile - split * per_split;
  constexpr int kRb = 4;  // row blocks per group
  const int grp = rem / (kRb * a.tbs), in = rem - grp * kRb * a.tbs;
  const int rows = a.rbs - grp * kRb < kRb ? a.rbs - grp * kRb : kRb;
  tbk = in / rows;
  rb = grp * kRb + (in - tbk * rows);
}

// Waves form kWT groups of 4: wave w takes row tiles kRT (w % 4) .. + kRT - 1 and token
// tiles kTT (w / 4) .. + kTT - 1, so the workgroup (256 kWT threads) owns 64 kRT rows and
// 16 kTT kWT tokens. With kWT = 2 each SIMD runs two waves, one's VALU work beside the
// other's MFMAs.
template <int kFmt, int kWT, int kTT, int kRT>
__global__ __launch_bounds__(256 * kWT) void oproj_mfma_kernel(MxArgs a) {
  constexpr bool kQ6 = kFmt == kMQ6K;
  using F = WFmt<kFmt>;
  constexpr int kThreads = 256 * kWT;
  constexpr int kTTg = kTT * kWT;                     // token tiles of the workgroup
  constexpr int kRows = 64 * kRT, kTok = 16 * kTTg;
  constexpr int kWTotal = kRows * F::kUnits;          // weight units of one superblock
  constexpr int kWPer = (kWTotal + kThreads - 1) / kThreads;  // per thread
  constexpr int kAPer = 4 * kTTg / kWT;               // token-fragment units per thread
  static_assert(kAPer * kThreads == kTTg * 1024, "token fragments split evenly");
  __shared__ u4 As[kTTg][8][2][64];                   // [token tile][K-step][hi, lo][lane]
  __shared__ h4 Xs[kThreads / 64][64];                // [token tile (spares past kTTg)][lane]
  __shared__ __attribute__((aligned(16))) uint8_t Wr[kRows * F::kRowImg + 16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave & 3, tt0 = kTT * (wave >> 2);  // row group, first token tile
  int split, rb, tbk;
  tile_of(a, (int)blockIdx.x, (int)gridDim.x, split, rb, tbk);
  const int s0 = split * a.sb_per_split;
  const int s1 = s0 + a.sb_per_split < a.SB ? s0 + a.sb_per_split : a.SB;
  const int r16 = lane & 15, g = lane >> 4;
  const int row0 = rb * kRows;

  // the next superblock's data in flight: token fragments, sub-block sums and weights,
  // every load outside any branch (past-the-end units re-read the last one), stored to
  // LDS only at the end of a step
  u4 pa[kAPer], pw[kWPer];
  h4 px = h4{0, 0, 0, 0};
  uint32_t t0 = 0, t1 = 0, tsh = 0;  // Q6K: row tid's image dword 52 (raw halves, shift)
  auto fetch = [&](int s) {
#pragma unroll
    for (int k = 0; k < kWPer; ++k) {
      const int u = tid + kThreads * k < kWTotal ? tid + kThreads * k : kWTotal - 1;
      pw[k] = load_unit<kFmt>(a.w, a.row_bytes, row0, a.N, s, u);
    }
    if constexpr (kQ6) {
      load_q6_tail(a.w, a.row_bytes, row0, a.N, s, tid < kRows ? tid : kRows - 1, t0, t1);
      tsh = (uint32_t)((210 * (int64_t)s) & 3);
    }
    // token fragments: unit v = tid + kThreads i of the kTTg * 1024: (token tile v / 1024,
    // hi / lo (v / 512) % 2, token m, piece p of the superblock's 32 eight-input pieces);
    // m runs fastest, so that a wave reads 64 contiguous bytes of 16 token rows and
    // writes one whole 1 KB fragment row of LDS
#pragma unroll
    for (int i = 0; i < kAPer; ++i) {
      const int v = tid + kThreads * i, rest = v & 511, m = rest & 15, p = rest >> 4;
      const int64_t row = (int64_t)(kTok * tbk + 16 * (v >> 10) + m) * (a.KB << 2);
      pa[i] = ((v >> 9) & 1 ? a.xl : a.xh)[row + 32 * s + p];
    }
    if constexpr (!kQ6) {
      const int u = tid & (64 * kTTg - 1);  // threads past 64 kTTg load copies
      const int m = u & 15, gg = (u >> 4) & 3, tt = u >> 6;
      px = a.xs[((int64_t)(kTok * tbk + 16 * tt + m) * a.SB + s) * 4 + gg];
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int k = 0; k < kWPer; ++k) {
      const int u = tid + kThreads * k, r = u / F::kUnits, p = u - r * F::kUnits;
      if (kWTotal % kThreads == 0 || u < kWTotal)
        *reinterpret_cast<u4 *>(Wr + r * F::kRowImg + 16 * p) = pw[k];
    }
    if constexpr (kQ6) {
      if (kRows == kThreads || tid < kRows)
        *reinterpret_cast<uint32_t *>(Wr + tid * F::kRowImg + 208) = tsh != 0 ? (t0 | (t1 << 16)) : t1;
    }
#pragma unroll
    for (int i = 0; i < kAPer; ++i) {
      const int v = tid + kThreads * i, rest = v & 511, m = rest & 15, p = rest >> 4;
      As[v >> 10][p >> 2][(v >> 9) & 1][m + 16 * (p & 3)] = pa[i];
    }
    if constexpr (!kQ6) Xs[tid >> 6][tid & 63] = px;
  };

  f4 fin[kTT][kRT];
#pragma unroll
  for (int tt = 0; tt < kTT; ++tt)
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt) fin[tt][rt] = f4{0.f, 0.f, 0.f, 0.f};

  fetch(s0);
  store();
  __syncthreads();
  for (int s = s0; s < s1; ++s) {
    // the next superblock's loads (the last step re-reads its own, unused), kept ahead of
    // the compute: without the barrier the scheduler sinks them below it to save
    // registers, and every step then waits for memory
    fetch(s + 1 < s1 ? s + 1 : s);
    __builtin_amdgcn_sched_barrier(0);
    // this lane's row in each of the wave's row tiles
    const uint8_t *img[kRT];
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt) img[rt] = Wr + (wr * 16 * kRT + rt * 16 + r16) * F::kRowImg;
    float dd[kRT], dm[kRT];
    uint32_t scb[kRT][2], mcb[kRT][2];  // Q4K/Q5K: scale / min codes as bytes
    uint32_t q6s[kRT][2];               // Q6K: the scales of this lane's sub-blocks
    int sh = 0;                         // Q6K: the block's offset in its image (0 or 2)
    if constexpr (kQ6) {
      // the image starts at the block's dword-aligned start: the same shift for all rows
      // (row_bytes is a multiple of 16)
      sh = (int)((210 * (int64_t)s) & 3);
    }
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt) {
      if constexpr (kQ6) {
        uint32_t sc4[4], dw[1];
        img_dwords(img[rt], 192 + sh, sc4);
        img_dwords(img[rt], 208 + sh, dw);
        // lane group g uses scales 2 j + g / 2 (j = 0..7): bytes g / 2, g / 2 + 2, ..
        const int o = 8 * (g >> 1);
        q6s[rt][0] = __builtin_amdgcn_perm(sc4[1], sc4[0], 0x06040200u + 0x01010101u * (o >> 3));
        q6s[rt][1] = __builtin_amdgcn_perm(sc4[3], sc4[2], 0x06040200u + 0x01010101u * (o >> 3));
        dd[rt] = h2f(dw[0] & 0xFFFFu);
        dm[rt] = 0.0f;
      } else {
        const u4 hdr = *reinterpret_cast<const u4 *>(img[rt]);
        const uint32_t s0w = hdr[1], s1w = hdr[2], s2w = hdr[3];
        scb[rt][0] = s0w & 0x3F3F3F3Fu;
        mcb[rt][0] = s1w & 0x3F3F3F3Fu;
        scb[rt][1] = (s2w & 0x0F0F0F0Fu) | ((s0w >> 2) & 0x30303030u);
        mcb[rt][1] = ((s2w >> 4) & 0x0F0F0F0Fu) | ((s1w >> 2) & 0x30303030u);
        dd[rt] = h2f(hdr[0] & 0xFFFFu);
        dm[rt] = h2f(hdr[0] >> 16) * 64.0f;  // the sums were scaled by 2^-6
      }
    }
    f4 acc[kTT][kRT];
#pragma unroll
    for (int tt = 0; tt < kTT; ++tt)
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) acc[tt][rt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      h8 ah[kTT], al[kTT];
#pragma unroll
      for (int tt = 0; tt < kTT; ++tt) {
        ah[tt] = __builtin_bit_cast(h8, As[tt0 + tt][j][0][lane]);
        al[tt] = __builtin_bit_cast(h8, As[tt0 + tt][j][1][lane]);
      }
      // the K-step's B fragments of all the wave's row tiles first, then the MFMAs ordered
      // so that the two that update one accumulator are kTT * kRT apart
      constexpr int kPl = kQ6 ? 2 : 1;
      h8 bf[kRT][kPl];
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) {
        if constexpr (kQ6) {
          // K-step j: half h = j / 4, group gg = j % 4; inputs 32 j + 8 g + i have scale
          // 2 j + g / 2 and codes from low-nibble bytes 64 h + 32 (gg & 1) + 8 g + i
          // (nibble gg / 2) and bits 2 gg of bit-pair bytes 128 + 32 h + 8 g + i
          const int h = j >> 2, gg = j & 3;
          uint32_t lo[2], hb[2];
          img_dwords(img[rt], 64 * h + 32 * (gg & 1) + 8 * g + sh, lo);
          img_dwords(img[rt], 128 + 32 * h + 8 * g + sh, hb);
          uint32_t x[2];
#pragma unroll
          for (int k = 0; k < 2; ++k)
            x[k] = ((lo[k] >> (4 * (gg >> 1))) & 0x0F0F0F0Fu) |
                   (((hb[k] >> (2 * gg)) & 0x03030303u) << 4);
          const int sc = (int)(int8_t)(uint8_t)(q6s[rt][j >> 2] >> (8 * (j & 3)));
          const float sl = (float)(sc & 15), shv = (float)(sc >> 4);
          bf[rt][0] = scaled_codes(x[0], x[1], h2_splat(sl), h2_splat(-1056.0f * sl));
          // 16 sh (q - 32): multiples of 16 up to 4096, exact
          bf[rt][kPl - 1] = scaled_codes(x[0], x[1], h2_splat(shv), h2_splat(-1056.0f * shv)) *
                            (_Float16)16.0f;
        } else {
          constexpr int kNib = kFmt == kMQ5K ? 48 : 16;
          const int c = j >> 1, hn = 4 * (j & 1);
          const uint2 nb = *reinterpret_cast<const uint2 *>(img[rt] + kNib + 32 * c + 8 * g);
          uint32_t x0 = (nb.x >> hn) & 0x0F0F0F0Fu, x1 = (nb.y >> hn) & 0x0F0F0F0Fu;
          if constexpr (kFmt == kMQ5K) {
            const uint2 qh = *reinterpret_cast<const uint2 *>(img[rt] + 16 + 8 * g);
            x0 |= ((qh.x >> j) & 0x01010101u) << 4;
            x1 |= ((qh.y >> j) & 0x01010101u) << 4;
          }
          const float sc = (float)((scb[rt][j >> 2] >> (8 * (j & 3))) & 0xFFu);
          bf[rt][0] = scaled_codes(x0, x1, h2_splat(sc), h2_splat(-1024.0f * sc));
        }
      }
#pragma unroll
      for (int pl = 0; pl < kPl; ++pl)
#pragma unroll
        for (int hl = 0; hl < 2; ++hl)
#pragma unroll
          for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
            for (int tt = 0; tt < kTT; ++tt)
              acc[tt][rt] = mfma32(hl ? al[tt] : ah[tt], bf[rt][pl], acc[tt][rt]);
    }
    if constexpr (!kQ6) {
      // min term: sum_j m_j xsum_j, k 0-7 the hi sums and 8-15 the lo sums
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) {
        const uint32_t mw = mcb[rt][g & 1];
        const h4 bm = h4{(_Float16)(float)(mw & 0xFFu), (_Float16)(float)((mw >> 8) & 0xFFu),
                         (_Float16)(float)((mw >> 16) & 0xFFu), (_Float16)(float)(mw >> 24)};
#pragma unroll
        for (int tt = 0; tt < kTT; ++tt) {
          const f4 am = mfma16(Xs[tt0 + tt][lane], bm, f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
          for (int i = 0; i < 4; ++i)
            fin[tt][rt][i] += dd[rt] * acc[tt][rt][i] - dm[rt] * am[i];
        }
      }
    } else {
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
        for (int tt = 0; tt < kTT; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) fin[tt][rt][i] += dd[rt] * acc[tt][rt][i];
    }
    __syncthreads();  // every wave is done with this superblock's LDS
    store();          // the last step's copy is never read
    __syncthreads();
  }
  // D layout: lane holds rows (tokens) 4 g + i of the tile, column (weight row) lane & 15
  float *dst = a.S == 1 ? a.out : a.part + (int64_t)split * a.T * a.N;
#pragma unroll
  for (int tt = 0; tt < kTT; ++tt)
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt) {
      const int n = row0 + wr * 16 * kRT + rt * 16 + r16;
      if (n >= a.N) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = tbk * kTok + 16 * (tt0 + tt) + 4 * g + i;
        if (t >= a.T) continue;
        dst[(int64_t)t * a.N + n] = a.S == 1 ? a.inv[t] * fin[tt][rt][i] : fin[tt][rt][i];
      }
    }
}

// out[t][n] = 2^-e_t * sum over splits in order: grid y over tokens, x over the row in
// float4 (N % 4 == 0) or single floats
__global__ __launch_bounds__(256) void oproj_reduce_kernel(const float *part, const float *inv,
                                                            float *out, int T, int N, int S) {
  const int64_t plane = (int64_t)T * N;
  for (int t = blockIdx.y; t < T; t += gridDim.y) {
    const float f = inv[t];
    const int64_t r0 = (int64_t)t * N;
    if ((N & 3) == 0) {
      for (int c = blockIdx.x * 256 + threadIdx.x; c < (N >> 2); c += gridDim.x * 256) {
        float4 s = reinterpret_cast<const float4 *>(part + r0)[c];
        for (int k = 1; k < S; ++k) {
          const float4 v = reinterpret_cast<const float4 *>(part + k * plane + r0)[c];
          s.x += v.x;
          s.y += v.y;
          s.z += v.z;
          s.w += v.w;
        }
        reinterpret_cast<float4 *>(out + r0)[c] = float4{f * s.x, f * s.y, f * s.z, f * s.w};
      }
    } else {
      for (int c = blockIdx.x * 256 + threadIdx.x; c < N; c += gridDim.x * 256) {
        float s = part[r0 + c];
        for (int k = 1; k < S; ++k) s += part[k * plane + r0 + c];
        out[r0 + c] = f * s;
      }
    }
  }
}


}  // namespace

int launch_oproj_mfma(const float *attn, const float *gate, const uint8_t *w, int w_type,
                      float *out, int batch, int in_dim, int out_dim, Workspace &ws,
                      hipStream_t s) {
  if (w_type != kMQ4K && w_type != kMQ5K && w_type != kMQ6K)
    return set_error(PKV_ERR_UNSUPPORTED, "batched o_proj: weight type must be Q4K, Q5K or Q6K");
  if (in_dim % 4096 != 0 || in_dim > 8192)
    return set_error(PKV_ERR_UNSUPPORTED, "batched o_proj: in_dim must be 4096 or 8192");
  for (const void *p : {(const void *)attn, (const void *)gate, (const void *)w})
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
      return set_error(PKV_ERR_ARG, "attn, gate and the weights must be 16-byte aligned");
  const int T = batch, N = out_dim, K = in_dim;
  // tile: 32 tokens x 256 rows per workgroup of 4 waves (32 x 64 per wave)
  const int tok = 32, rows = 256;
  const int T_pad = (T + tok - 1) / tok * tok;
  const int KB = K / 32, SB = K / 256;
  const int64_t row_bytes = (int64_t)SB * (w_type == kMQ4K ? 144 : w_type == kMQ5K ? 176 : 210);
  const int rbs = (N + rows - 1) / rows, tbs = T_pad / tok;
  if ((int64_t)rbs * tbs * SB > (1 << 30))
    return set_error(PKV_ERR_ARG, "batch too large for the batched o_proj");
  int S = kMxTargetWGs / (rbs * tbs);
  S = S < 1 ? 1 : (S > SB ? SB : S);
  const int per = (SB + S - 1) / S;
  S = (SB + per - 1) / per;  // no empty split
  const size_t xhl_bytes = (size_t)T_pad * K * 2, xs_bytes = (size_t)T_pad * SB * 32;
  const size_t inv_bytes = (size_t)T_pad * 4;
  const size_t part_bytes = S > 1 ? (size_t)S * T * N * 4 : 0;
  const size_t off_xl = xhl_bytes, off_xs = 2 * xhl_bytes, off_inv = off_xs + xs_bytes;
  const size_t off_part = (off_inv + inv_bytes + 255) / 256 * 256;
  if (int rc = ws.reserve(off_part + part_bytes)) return rc;
  uint8_t *base = static_cast<uint8_t *>(ws.ptr);
  XprepArgs xa{attn, gate, T, K, reinterpret_cast<u4 *>(base), reinterpret_cast<u4 *>(base + off_xl),
               reinterpret_cast<h4 *>(base + off_xs), reinterpret_cast<float *>(base + off_inv)};
  if (K == 4096)
    hipLaunchKernelGGL(oproj_xprep_kernel<2>, dim3((unsigned)T_pad), dim3(256), 0, s, xa);
  else
    hipLaunchKernelGGL(oproj_xprep_kernel<4>, dim3((unsigned)T_pad), dim3(256), 0, s, xa);
  PKV_HIP(hipGetLastError());
  MxArgs ma{reinterpret_cast<const u4 *>(base), reinterpret_cast<const u4 *>(base + off_xl),
            reinterpret_cast<const h4 *>(base + off_xs),
            reinterpret_cast<const float *>(base + off_inv), w, row_bytes,
            reinterpret_cast<float *>(base + off_part), out, T, N, KB, SB, per, S, rbs, tbs};
  const dim3 grid((unsigned)(rbs * tbs * S));
#define PKV_MX(FMT) hipLaunchKernelGGL((oproj_mfma_kernel<FMT, 1, 2, 4>), grid, dim3(256), 0, s, ma)
  switch (w_type) {
    case kMQ4K: PKV_MX(kMQ4K); break;
    case kMQ5K: PKV_MX(kMQ5K); break;
    default: PKV_MX(kMQ6K); break;
  }
#undef PKV_MX
  PKV_HIP(hipGetLastError());
  if (S > 1) {
    const int per_row = N % 4 == 0 ? N / 4 : N;
    const dim3 rgrid((unsigned)((per_row + 255) / 256), (unsigned)(T < 65535 ? T : 65535));
    hipLaunchKernelGGL(oproj_reduce_kernel, rgrid, dim3(256), 0, s,
                       reinterpret_cast<const float *>(base + off_part),
                       reinterpret_cast<const float *>(base + off_inv), out, T, N, S);
    PKV_HIP(hipGetLastError());
  }
  return PKV_OK;
}

}  // namespace pkv
