// Q8_0 operand builders shared by the MFMA kernels over Q8_0 caches (prefill chunk and
// decode), gfx950. A Q8_0 row of a 256-dim head is 8 blocks of {f16 d, 32 x int8}
// (272 bytes): element e is int8 * d of block e / 32 (BlockQ8_0::to_float).
// Include-only; every symbol has internal linkage.
#pragma once
#include "pkv_mfma_common.hpp"

namespace pkv {
namespace {

constexpr int kQ8RowB = 272;  // bytes of one head's Q8_0 row (8 x 34)

// Block-local key of row r of tile t (the QK A layout): lane (n, g) of the QK result
// then holds keys 8g + 4t + i for row n.
__device__ __forceinline__ int q8_key(int r, int t) { return 8 * (r >> 2) + 4 * t + (r & 3); }

// Four int8 in a dword -> two dwords of two fp16 each, exactly: the bytes, offset by 128,
// become the low bytes of fp16 1024 + u (exponent byte 0x64), then 1152 is subtracted.
__device__ __forceinline__ void i8x4_to_h4(uint32_t w, h2 &lo, h2 &hi) {
  const uint32_t u = w ^ 0x80808080u;
  const h2 k = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  lo = as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) + k;
  hi = as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) + k;
}

// {fp16(a0 - c0), fp16(a1 - c1)} for the fp16 halves c0, c1 of cw, each rounded once
// from the exact f32 difference (v_fma_mix). The words are only stored to LDS (no MFMA
// reads them), so no wait states follow.
__device__ __forceinline__ uint32_t lo_pair(float a0, float a1, uint32_t cw) {
  uint32_t d;
  asm("v_fma_mixlo_f16 %0, %1, 1.0, -%3 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixhi_f16 %0, %2, 1.0, -%3 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
      : "=&v"(d)
      : "v"(a0), "v"(a1), "v"(cw));
  return d;
}

// The PV B fragments of unit vw = 2 h + kHl (four 16-column tiles T = 8 h + kHl + 2 b,
// b = 0..3) for 32 keys whose rows start every `row_words` dwords at `rows`: the columns
// follow the decode kernels' tile order (column n of tile T is element tile_e(T, n)), so
// lane (n, g) takes, for each of keys 8 g .. 8 g + 7, the four codes 4 (n & 7) .. + 3 of
// block j = 4 h + 2 (n >> 3) + kHl (one dword, two bytes past a dword boundary for even
// j), code b going to tile 8 h + kHl + 2 b. Each value int8 * d (at most 18 significant
// bits, exact in f32: the code + 128 times d, minus 128 d, in one fma) becomes an fp16 hi
// part and the exact lo remainder: wh[b - kB0][p] / wl[b - kB0][p] hold keys 8 g + 2 p,
// + 1, for the codes b = kB0 .. kB0 + kNB - 1 (all four by default).
template <int kHl, int kB0 = 0, int kNB = 4>
__device__ __forceinline__ void q8_v_words(const uint32_t *rows, int row_words, int h, int lane,
                                           uint32_t (&wh)[kNB][4], uint32_t (&wl)[kNB][4]) {
  const int n = lane & 15, g = lane >> 4;
  const int j = 4 * h + 2 * (n >> 3) + kHl;
  const int cw = (34 * j + 2 + 4 * (n & 7)) >> 2;  // first dword of the four codes
  const int dw = (34 * j) >> 2;                     // dword of d: low half (even j) or high
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    float v[2][kNB];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const uint32_t *row = rows + (8 * g + 2 * p + kk) * row_words;
      uint32_t w = kHl ? row[cw] : __builtin_amdgcn_alignbyte(row[cw + 1], row[cw], 2);
      w ^= 0x80808080u;  // code + 128 in each byte
      const uint32_t dd = row[dw];
      const float d = h2f(kHl ? (dd >> 16) : (dd & 0xFFFF)), nd = -128.0f * d;
#pragma unroll
      for (int b = 0; b < kNB; ++b)
        v[kk][b] = fmaf((float)((w >> (8 * (b + kB0))) & 0xFFu), d, nd);
    }
#pragma unroll
    for (int b = 0; b < kNB; ++b) {
      wh[b][p] = as_u(h2{(_Float16)v[0][b], (_Float16)v[1][b]});
      wl[b][p] = lo_pair(v[0][b], v[1][b], wh[b][p]);
    }
  }
}

}  // namespace
}  // namespace pkv
