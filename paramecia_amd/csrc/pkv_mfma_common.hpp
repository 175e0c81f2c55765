// Building blocks shared by the MFMA attention kernels over Q4K rows (decode and
// prefill): vector types, the exact fp16 operand tricks, GGML scale decoding, the LDS
// staging layout of 32-key blocks with its buffer_load ... lds issue, and cross-lane
// reductions. Include-only; every symbol has internal linkage.
#pragma once
#include "pkv_decode_split.hpp"
#include "pkv_internal.hpp"
#include "pkv_scalar.hpp"

namespace pkv {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kBlk = 32;  // keys per staged block
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kClampL2 = 100.0f * 1.4426950408889634f;  // +-100 nats in log2 units

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
// {fp16(a0 - c0), fp16(a1 - c1)} with c0, c1 the fp16 halves of cw: v_fma_mix computes
// a * 1.0 - c in f32 (exact for c = fp16(a) or 0) and rounds once to fp16. The words feed
// MFMA operands. The compiler inserts the wait states between a VALU write and an MFMA read
// only for instructions it can see, so the asm ends with its own (s_nop 4: five wait
// states, more than a VALU write needs before an MFMA reads the register); its inputs are
// VALU results, never MFMA results. Written in C instead, the compiler fused the caller's
// product into a v_fma_mix with two f32 multiplicands, which lost about ten bits of the
// hi + lo pair; and an inline-asm v_fma_mix that read an MFMA result three instructions
// after the MFMA returned the previous partial sum, which is why asm here takes no MFMA
// results.
__device__ __forceinline__ uint32_t fp16_sub2(float a0, float a1, uint32_t cw) {
  uint32_t d;
  asm("v_fma_mixlo_f16 %0, %1, 1.0, -%3 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixhi_f16 %0, %2, 1.0, -%3 op_sel:[0,0,1] op_sel_hi:[0,0,1]\n\t"
      "s_nop 4"
      : "=&v"(d)
      : "v"(a0), "v"(a1), "v"(cw));
  return d;
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

// ---- LDS staging of 32-key blocks. One tensor (K or V) of one KV head: the 16-byte
// header of row R at hdr[R], and the row's eight 16-byte nibble pieces at
// nib[8R + (piece ^ swz(R))]. The XOR swizzle makes the row-wise K reads of phase Q
// conflict-free and keeps the transposed V reads of phase P at two ways.
struct TensorStage {
  u4 hdr[kBlk];
  u4 nib[8 * kBlk];
};
struct Stage {
  TensorStage k, v;
};
constexpr int kLoadsPerStage = 12;  // 4 x dwordx4 (pieces) + 2 x dword (headers), K and V
__device__ __forceinline__ int swz(int R) { return ((R >> 1) & 1) | (((R >> 3) & 3) << 1); }

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

// One lane's part of staging a block, as byte offsets from the block's first row
// (the same for K and V, whose rows share the stride). The block's own offset is
// added in the voffset operand, so the buffer range check covers the whole address.
struct LoadPlan {
  uint32_t nib[4];  // dwordx4 load i: slot 64 i + lane
  uint32_t hdr[2];  // dword load j: dword (lane & 3) of header 16 j + lane / 4
};

__device__ __forceinline__ LoadPlan make_plan(int lane, uint32_t rs_t) {
  LoadPlan P;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int slot = 64 * i + lane, R = slot >> 3;
    const int piece = (slot & 7) ^ swz(R);
    P.nib[i] = (uint32_t)R * rs_t + 16u + 16u * (uint32_t)piece;
  }
#pragma unroll
  for (int j = 0; j < 2; ++j)
    P.hdr[j] = (uint32_t)(16 * j + (lane >> 2)) * rs_t + 4u * (uint32_t)(lane & 3);
  return P;
}

// Stage one block (K and V) into LDS: 12 buffer_load ... lds, written from inline asm
// so that the compiler's wait-count pass does not serialise later LDS reads behind
// them; the kernel places its own s_waitcnt vmcnt before a stage is read. M0 holds
// the LDS destination of each load (lane l writes M0 + 16 l, or M0 + 4 l for dwords);
// one wait state separates an M0 write from the load that reads it.
__device__ __forceinline__ void issue_stage(Stage *st, const LoadPlan &P, u4s rk, u4s rv,
                                            uint32_t boff) {
  const uint32_t kn = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)((PKV_LDS void *)&st->k.nib[0]));
  const uint32_t kh = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)((PKV_LDS void *)&st->k.hdr[0]));
  const uint32_t vn = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)((PKV_LDS void *)&st->v.nib[0]));
  const uint32_t vh = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)((PKV_LDS void *)&st->v.hdr[0]));
  const uint32_t o0 = P.nib[0] + boff, o1 = P.nib[1] + boff, o2 = P.nib[2] + boff,
                 o3 = P.nib[3] + boff, h0 = P.hdr[0] + boff, h1 = P.hdr[1] + boff;
  uint32_t saved;
  asm volatile(
      "s_nop 4\n\t"  // VALU-written SGPRs (v_readfirstlane) read by VMEM: 5 wait states
      "s_mov_b32 %[sv], m0\n\t"
      "s_mov_b32 m0, %[kn]\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o0], %[rk], 0 offen lds\n\t"
      "s_add_u32 m0, %[kn], 0x400\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o1], %[rk], 0 offen lds\n\t"
      "s_add_u32 m0, %[kn], 0x800\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o2], %[rk], 0 offen lds\n\t"
      "s_add_u32 m0, %[kn], 0xc00\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o3], %[rk], 0 offen lds\n\t"
      "s_mov_b32 m0, %[kh]\n\ts_nop 0\n\t"
      "buffer_load_dword %[h0], %[rk], 0 offen lds\n\t"
      "s_add_u32 m0, %[kh], 0x100\n\ts_nop 0\n\t"
      "buffer_load_dword %[h1], %[rk], 0 offen lds\n\t"
      "s_mov_b32 m0, %[vn]\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o0], %[rv], 0 offen lds\n\t"
      "s_add_u32 m0, %[vn], 0x400\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o1], %[rv], 0 offen lds\n\t"
      "s_add_u32 m0, %[vn], 0x800\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o2], %[rv], 0 offen lds\n\t"
      "s_add_u32 m0, %[vn], 0xc00\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o3], %[rv], 0 offen lds\n\t"
      "s_mov_b32 m0, %[vh]\n\ts_nop 0\n\t"
      "buffer_load_dword %[h0], %[rv], 0 offen lds\n\t"
      "s_add_u32 m0, %[vh], 0x100\n\ts_nop 0\n\t"
      "buffer_load_dword %[h1], %[rv], 0 offen lds\n\t"
      "s_mov_b32 m0, %[sv]"
      : [sv] "=&s"(saved)
      : [kn] "s"(kn), [kh] "s"(kh), [vn] "s"(vn), [vh] "s"(vh), [o0] "v"(o0), [o1] "v"(o1),
        [o2] "v"(o2), [o3] "v"(o3), [h0] "v"(h0), [h1] "v"(h1), [rk] "s"(rk), [rv] "s"(rv)
      : "memory", "scc");
}

// The resource r advanced by off <= its record count: base + off and the records past
// the new base, so that a lane's voffset alone is range checked. Plain scalar
// arithmetic (a saturating subtract would be a vector instruction).
__device__ __forceinline__ u4s rsrc_advance(u4s r, uint32_t off) {
  const uint64_t b = (((uint64_t)r.y << 32) | r.x) + off;  // r.y: address bits 32-47, stride 0
  u4s o;
  o.x = (uint32_t)b;
  o.y = (uint32_t)(b >> 32);
  o.z = r.z - off;
  o.w = r.w;
  return o;
}

// issue_stage with a wave-uniform LDS byte address of the Stage and the block's offset
// already in the resources: no vector work per issue. K: headers at +0, pieces at
// +0x200; V: headers at +0x1200, pieces at +0x1400. The loads go out in the order the
// block is read (K headers, K pieces, V headers, V pieces), so the data read first has
// landed longest when the stage's vmcnt wait completes.
__device__ __forceinline__ void issue_stage_at(uint32_t base, const LoadPlan &P, u4s rk, u4s rv) {
  static_assert(sizeof(TensorStage) == 0x1200 && sizeof(Stage) == 0x2400, "stage layout");
  uint32_t saved;
  asm volatile(
      "s_nop 4\n\t"  // VALU-written SGPRs (v_readfirstlane) read by VMEM: 5 wait states
      "s_mov_b32 %[sv], m0\n\t"
      "s_mov_b32 m0, %[b]\n\ts_nop 0\n\t"
      "buffer_load_dword %[h0], %[rk], 0 offen lds\n\t"
      "s_add_u32 m0, %[b], 0x100\n\ts_nop 0\n\t"
      "buffer_load_dword %[h1], %[rk], 0 offen lds\n\t"
      "s_add_u32 m0, %[b], 0x200\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o0], %[rk], 0 offen lds\n\t"
      "s_add_u32 m0, %[b], 0x600\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o1], %[rk], 0 offen lds\n\t"
      "s_add_u32 m0, %[b], 0xa00\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o2], %[rk], 0 offen lds\n\t"
      "s_add_u32 m0, %[b], 0xe00\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o3], %[rk], 0 offen lds\n\t"
      "s_add_u32 m0, %[b], 0x1200\n\ts_nop 0\n\t"
      "buffer_load_dword %[h0], %[rv], 0 offen lds\n\t"
      "s_add_u32 m0, %[b], 0x1300\n\ts_nop 0\n\t"
      "buffer_load_dword %[h1], %[rv], 0 offen lds\n\t"
      "s_add_u32 m0, %[b], 0x1400\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o0], %[rv], 0 offen lds\n\t"
      "s_add_u32 m0, %[b], 0x1800\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o1], %[rv], 0 offen lds\n\t"
      "s_add_u32 m0, %[b], 0x1c00\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o2], %[rv], 0 offen lds\n\t"
      "s_add_u32 m0, %[b], 0x2000\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %[o3], %[rv], 0 offen lds\n\t"
      "s_mov_b32 m0, %[sv]"
      : [sv] "=&s"(saved)
      : [b] "s"(base), [o0] "v"(P.nib[0]), [o1] "v"(P.nib[1]), [o2] "v"(P.nib[2]),
        [o3] "v"(P.nib[3]), [h0] "v"(P.hdr[0]), [h1] "v"(P.hdr[1]), [rk] "s"(rk), [rv] "s"(rv)
      : "memory", "scc");
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

// Sum over lanes l and l ^ 32 of x (lanes 0-31) and of y (lanes 32-63) with one swap:
// v_permlane32_swap(x, y) exchanges x's upper 32 lanes with y's lower 32 lanes.
__device__ __forceinline__ float pair_sum32(float x, float y) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x),
                                                  __builtin_bit_cast(uint32_t, y), false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}

__device__ __forceinline__ float xsum32(float x) {  // x of lanes l and l ^ 32, summed
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}


}  // namespace
}  // namespace pkv
