// Quantize-on-append and dequantize kernels for the packed KV rows.
//
// Reference: PreallocatedQuantizedKvCache::append_quantized
// (paramecia-model/src/qwen3_next.rs:431-509) quantizes the new [b, h, n, d] K/V on
// the CPU with candle's QTensor::quantize and memcpy's the rows at
// seq_len*b*h*bytes_per_row; get_kv (qwen3_next.rs:520-575) dequantizes them.
// Here both run on the GPU, writing/reading the same seq-major rows in HBM.
//
// Bit-exactness: every a*b+c below must round twice like the Rust code, so
// contraction is off for this whole file, divisions are IEEE (hipcc's default), and
// each Q4K sub-block's sums run sequentially in one lane.
#pragma clang fp contract(off)

#include "pkv_internal.hpp"
#include "pkv_scalar.hpp"
#include "pkv_q4k_lanes.hpp"

namespace pkv {
namespace {

struct AppendArgs {
  const float *src[2];  // k, v: [batch, heads, n, head_dim]
  uint8_t *dst[2];      // K, V row buffers (paged: the pool's K and V page planes)
  int batch, heads, head_dim, padded;
  int64_t n, t0;
  int64_t bpr;
  // Paged rows (page_tab non-null): token t lives in page page_tab[t >> page_lg], row
  // t & (2^page_lg - 1) of that page, each page page_bytes long in each plane
  const int32_t *page_tab;
  int page_lg;
  int64_t page_bytes;
  // One token into each of `batch` paged sequences (row_mode): row (b, h) at byte
  // row_off[b] + h * bpr of each plane
  int row_mode;
  int64_t row_off[kAppendSeqs];
};

// Source element e (< padded) of new row (t, b, h); zero padding past head_dim.
__device__ __forceinline__ float load_elem(const float *src, const AppendArgs &a, int64_t t,
                                           int b, int h, int e) {
  if (e >= a.head_dim) return 0.0f;
  return src[(((int64_t)b * a.heads + h) * a.n + t) * a.head_dim + e];
}

__device__ __forceinline__ int64_t dst_row(const AppendArgs &a, int64_t t, int b, int h) {
  return ((a.t0 + t) * a.batch + b) * a.heads + h;
}
// The destination row of new token t (batch row b, head h) in plane p (K 0, V 1).
__device__ __forceinline__ uint8_t *row_ptr(const AppendArgs &a, int p, int64_t t, int b, int h) {
  if (a.row_mode) return a.dst[p] + a.row_off[b] + (int64_t)h * a.bpr;
  if (a.page_tab != nullptr) {
    const int64_t tok = a.t0 + t, in_page = tok & ((int64_t(1) << a.page_lg) - 1);
    const int64_t pg = a.page_tab[tok >> a.page_lg];
    return a.dst[p] + pg * a.page_bytes + ((in_page * a.batch + b) * a.heads + h) * a.bpr;
  }
  return a.dst[p] + dst_row(a, t, b, h) * a.bpr;
}

// Lanes per Q4K sub-block in the throughput kernel (kL = 1, 2, 4) and the helpers that
// join a sub-block's kL lanes: all moves within a quad of lanes (DPP), exact.
template <int kL, int q>
__device__ __forceinline__ float group_bcast(float v) {  // lane q of the group's value
  if constexpr (kL == 1) {
    return v;
  } else {
    constexpr int ctrl = kL == 2 ? (q | (q << 2) | ((2 + q) << 4) | ((2 + q) << 6)) : q * 0x55;
    return u2f((uint32_t)__builtin_amdgcn_update_dpp(0, (int)f2u(v), ctrl, 0xF, 0xF, false));
  }
}
template <int kL, typename T, typename Op>
__device__ __forceinline__ T group_allreduce(T v, Op op) {  // order-free ops only
  if constexpr (kL >= 2) {
    const int o = __builtin_amdgcn_update_dpp(0, (int)__builtin_bit_cast(uint32_t, v), 0xB1, 0xF,
                                              0xF, false);  // quad_perm [1,0,3,2]
    v = op(v, __builtin_bit_cast(T, o));
  }
  if constexpr (kL >= 4) {
    const int o = __builtin_amdgcn_update_dpp(0, (int)__builtin_bit_cast(uint32_t, v), 0x4E, 0xF,
                                              0xF, false);  // quad_perm [2,3,0,1]
    v = op(v, __builtin_bit_cast(T, o));
  }
  return v;
}
// acc + term[0] + ... over the whole sub-block, in element order with one rounding per add:
// lane q of the group adds its E terms to the running sum, which every lane then takes
// from lane q (the other lanes' adds that step are discarded).
template <int kL, int q = 0>
struct GroupChain {
  template <int E>
  static __device__ __forceinline__ float run(const float (&term)[E], float acc) {
#pragma clang fp contract(off)
#pragma unroll
    for (int i = 0; i < E; ++i) acc += term[i];
    acc = group_bcast<kL, q>(acc);
    if constexpr (q + 1 < kL)
      return GroupChain<kL, q + 1>::run(term, acc);
    else
      return acc;
  }
};
template <int kL>
__device__ __forceinline__ bool group_any(bool c) {
  if constexpr (kL == 1) {
    return c;
  } else {
    const uint64_t bal = __ballot(c);
    const int base = (int)(threadIdx.x & 63) & ~(kL - 1);
    return ((bal >> base) & ((1u << kL) - 1)) != 0;
  }
}

// Q4K (BlockQ4K::from_float): 8 kL lanes per 256-element superblock. Lane (j, s) of the
// superblock holds elements [32 j + s E, 32 j + (s + 1) E) of sub-block j, E = 32 / kL.
// The sub-block fit is candle's make_qkx1_quants(nmax = 15, ntry = 5): levels are floats
// (small integers, exact), suml2 an integer-valued f32 (exact, any order), and the two
// other sums run in element order with one rounding per add, lane after lane through the
// group. The element-wise work of a pass is split kL ways and the sums are not, so kL = 1
// gives the fewest instructions per superblock (large appends) and kL = 2 or 4 the
// shortest instruction stream per wave (appends with too few superblocks to fill the GPU).
// Cross-lane work is limited to exact moves, max reductions and byte shuffles.
template <int kL>
__global__ __launch_bounds__(256) void q4k_append_kernel(AppendArgs a, int64_t units_per_tensor,
                                                         int nsb) {
  constexpr int E = 32 / kL;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t unit = gid / (8 * kL);
  const int r = (int)(gid & (8 * kL - 1));
  const int j = r / kL, s = r & (kL - 1);
  const int64_t total = 2 * units_per_tensor;
  const bool active = unit < total;
  if (!active) unit = total - 1;  // compute redundantly, store nothing
  const int p = (int)(unit / units_per_tensor);
  int64_t u = unit % units_per_tensor;
  const int sb = (int)(u % nsb);
  u /= nsb;
  const int h = (int)(u % a.heads);
  u /= a.heads;
  const int b = (int)(u % a.batch);
  const int64_t t = u / a.batch;

  float x[E];
  const int e0 = sb * 256 + 32 * j + s * E;
  const float *src = a.src[p];
  if ((a.head_dim & 3) == 0 && e0 + E <= a.head_dim) {
    const float4 *s4 = reinterpret_cast<const float4 *>(
        src + (((int64_t)b * a.heads + h) * a.n + t) * a.head_dim + e0);
#pragma unroll
    for (int i = 0; i < E / 4; ++i) {
      float4 f = s4[i];
      x[4 * i] = f.x;
      x[4 * i + 1] = f.y;
      x[4 * i + 2] = f.z;
      x[4 * i + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < E; ++i) x[i] = load_elem(src, a, t, b, h, e0 + i);
  }

  // Sub-block min and max in f32::total_cmp order (exact integer keys)
  int32_t kmin = total_key(x[0]), kmax = kmin;
#pragma unroll
  for (int i = 1; i < E; ++i) {
    const int32_t k = total_key(x[i]);
    kmin = k < kmin ? k : kmin;
    kmax = k > kmax ? k : kmax;
  }
  kmin = group_allreduce<kL>(kmin, [](int32_t p, int32_t q) { return p < q ? p : q; });
  kmax = group_allreduce<kL>(kmax, [](int32_t p, int32_t q) { return p > q ? p : q; });
  const auto from_key = [](int32_t k) {
    return u2f((uint32_t)(k ^ (int32_t)(((uint32_t)(k >> 31)) >> 1)));
  };
  const float mn = from_key(kmin), mx = from_key(kmax);

  float scale = 0.0f, mins = 0.0f;
  if (!(mx == mn)) {
    float L[E];
#pragma unroll
    for (int i = 0; i < E; ++i) L[i] = 0.0f;
    float min = fmin_rs(mn, 0.0f);
    float iscale = 15.0f / (mx - min);
    scale = 1.0f / iscale;
    // split fits unroll their passes (no level copies between passes); the one-lane fit
    // stays rolled, unrolled it needs 130 VGPRs and loses a wave per SIMD
    constexpr int kPassUnroll = kL > 1 ? 5 : 1;
#pragma unroll kPassUnroll
    for (int it = 0; it < 5; ++it) {
      float term[E];
      float suml2 = 0.0f;
      bool did_change = false;
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const float d = x[i] - min;
        const float li = (float)q4_level_i(iscale * d);
        did_change |= li != L[i];
        L[i] = li;
        term[i] = d * li;
        suml2 = __builtin_fmaf(li, li, suml2);  // exact
      }
      suml2 = group_allreduce<kL>(suml2, [](float p, float q) { return p + q; });  // exact
      const float sumlx = GroupChain<kL>::run(term, 0.0f);
      scale = sumlx / suml2;
#pragma unroll
      for (int i = 0; i < E; ++i) term[i] = x[i] - scale * L[i];
      const float sum = GroupChain<kL>::run(term, -0.0f);
      min = sum / 32.0f;
      if (min > 0.0f) min = 0.0f;
      iscale = 1.0f / scale;
      if (!group_any<kL>(did_change)) break;
    }
    mins = -min;
  }

  float max_scale = scale, max_min = mins;
#pragma unroll
  for (int o = kL; o < 8 * kL; o <<= 1) {
    max_scale = fmax_rs(max_scale, __shfl_xor(max_scale, o, 8 * kL));
    max_min = fmax_rs(max_min, __shfl_xor(max_min, o, 8 * kL));
  }
  max_scale = fmax_rs(max_scale, 0.0f);
  max_min = fmax_rs(max_min, 0.0f);
  const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
  const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
  int32_t ls32 = nearest_int(inv_scale * scale);
  int32_t lm32 = nearest_int(inv_min * mins);
  const uint32_t ls = (uint8_t)(ls32 < 63 ? ls32 : 63);
  const uint32_t lm = (uint8_t)(lm32 < 63 ? lm32 : 63);

  const uint16_t dh = f32_to_f16(max_scale / 63.0f);
  const uint16_t mh = f32_to_f16(max_min / 63.0f);

  // get_scale_min_k4(j) of the packed codes returns (ls, lm) for this sub-block.
  // Levels clamp(nearest_int((x + dm) / dd), 0, 15) with a correctly rounded division.
  // Fast path: q = (x + dm) * rcp(dd) is within about 2 ulp of the rounded quotient
  // (v_rcp_f32 within 1 ulp), so rint(q) is its nearest integer unless q lies within
  // 2^-12 of a half-integer (a possible tie); those elements, and every element when
  // rcp(dd) is not finite, take the IEEE division.
  constexpr int NW = (E + 7) / 8;  // nibble words: element i at bits 4 (i % 8) of word i / 8
  uint32_t Lw[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) Lw[w] = 0u;
  const float dd = f16_to_f32(dh) * (float)ls;
  if (dd != 0.0f) {
    const float dm = f16_to_f32(mh) * (float)lm;
    const float rdd = __builtin_amdgcn_rcpf(dd);
    const bool exact_all = !(__builtin_fabsf(rdd) < 3.0e38f);
    uint32_t slow = 0u;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const float q = (x[i] + dm) * rdd;
      const float r = __builtin_rintf(q);
      const bool near_tie = __builtin_fabsf(q - r) > 0.5f - 0x1p-12f;
      slow |= (near_tie || exact_all) ? (1u << i) : 0u;
      float l = (r > 0.0f) ? r : 0.0f;  // negatives, -0 and NaN -> 0
      l = (l < 15.0f) ? l : 15.0f;
      Lw[i >> 3] |= (uint32_t)l << (4 * (i & 7));
    }
    if (slow != 0u) {
#pragma unroll
      for (int i = 0; i < E; ++i) {
        if (slow & (1u << i)) {
          const int32_t l = q4_level_i((x[i] + dm) / dd);
          Lw[i >> 3] = (Lw[i >> 3] & ~(15u << (4 * (i & 7)))) | ((uint32_t)l << (4 * (i & 7)));
        }
      }
    }
  }

  // Header: d, dmin, and the 12 packed scale bytes, gathered from the 8 sub-blocks.
  uint32_t code = ls | (lm << 8);
  uint32_t codes[8];
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) codes[jj] = __shfl(code, jj * kL, 8 * kL);
  uint8_t sc[12];
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const uint32_t ls_lo = codes[jj] & 0xFF, lm_lo = codes[jj] >> 8;
    const uint32_t ls_hi = codes[jj + 4] & 0xFF, lm_hi = codes[jj + 4] >> 8;
    sc[jj] = (uint8_t)(ls_lo | ((ls_hi >> 4) << 6));
    sc[jj + 4] = (uint8_t)(lm_lo | ((lm_hi >> 4) << 6));
    sc[jj + 8] = (uint8_t)((ls_hi & 0xF) | ((lm_hi & 0xF) << 4));
  }

  // Nibbles: qs[32c + l] = L_{2c}[l] | L_{2c+1}[l] << 4. Lanes (2c, s) and (2c+1, s) own
  // l in [sE, sE + E): the even lane writes the first E/2 bytes, the odd lane the rest,
  // each taking the other half of its partner's nibbles (partner: lane ^ kL).
  constexpr int H = E / 2;             // nibbles (= bytes written) per lane
  constexpr int HW = (H + 7) / 8;      // words per half
  const bool odd = (j & 1) != 0;
  uint32_t lo[HW], hi[HW];
#pragma unroll
  for (int w = 0; w < HW; ++w) {
    uint32_t first, second;  // this lane's nibbles [0, H) and [H, E)
    if constexpr (H >= 8) {
      first = Lw[w];
      second = Lw[HW + w];
    } else {
      first = Lw[0] & ((1u << (4 * H)) - 1u);
      second = Lw[0] >> (4 * H);
    }
    const uint32_t recv = __shfl_xor(odd ? first : second, kL, 8 * kL);
    lo[w] = odd ? recv : first;
    hi[w] = odd ? second : recv;
  }
  constexpr int NB = H / 4;  // output words
  uint32_t outw[NB];
#pragma unroll
  for (int w = 0; w < NB; ++w) {
    const uint32_t l4 = lo[w / 2] >> (16 * (w & 1)), h4 = hi[w / 2] >> (16 * (w & 1));
    uint32_t v = 0;
#pragma unroll
    for (int bb = 0; bb < 4; ++bb) {
      const uint32_t ln = (l4 >> (4 * bb)) & 0xF, hn = (h4 >> (4 * bb)) & 0xF;
      v |= (ln | (hn << 4)) << (8 * bb);
    }
    outw[w] = v;
  }
  if (!active) return;
  uint8_t *blk = row_ptr(a, p, t, b, h) + (int64_t)sb * 144;
  uint8_t *qdst = blk + 16 + 32 * (j >> 1) + s * E + (odd ? H : 0);
  if constexpr (NB == 4) {
    *reinterpret_cast<uint4 *>(qdst) = uint4{outw[0], outw[1], outw[2], outw[3]};
  } else if constexpr (NB == 2) {
    *reinterpret_cast<uint2 *>(qdst) = uint2{outw[0], outw[1]};
  } else {
    *reinterpret_cast<uint32_t *>(qdst) = outw[0];
  }
  if (r == 0) {
    uint4 hd;
    hd.x = (uint32_t)dh | ((uint32_t)mh << 16);
    hd.y = (uint32_t)sc[0] | ((uint32_t)sc[1] << 8) | ((uint32_t)sc[2] << 16) | ((uint32_t)sc[3] << 24);
    hd.z = (uint32_t)sc[4] | ((uint32_t)sc[5] << 8) | ((uint32_t)sc[6] << 16) | ((uint32_t)sc[7] << 24);
    hd.w = (uint32_t)sc[8] | ((uint32_t)sc[9] << 8) | ((uint32_t)sc[10] << 16) | ((uint32_t)sc[11] << 24);
    *reinterpret_cast<uint4 *>(blk) = hd;
  }
}

// One workgroup per (tensor, token, batch, head, superblock); for appends of a few rows.
__global__ __launch_bounds__(256) void q4k_append_small_kernel(AppendArgs a, int nsb) {
  __shared__ Q4kScratch scr;
  int64_t u = blockIdx.x;
  const int sb = (int)(u % nsb);
  u /= nsb;
  const int h = (int)(u % a.heads);
  u /= a.heads;
  const int b = (int)(u % a.batch);
  u /= a.batch;
  const int64_t t = u % a.n;
  const int p = (int)(u / a.n);
  const float x = load_elem(a.src[p], a, t, b, h, sb * 256 + (int)threadIdx.x);
  uint8_t *blk = row_ptr(a, p, t, b, h) + (int64_t)sb * 144;
  q4k_quantize_superblock_lanes(x, blk, &scr, (int)threadIdx.x);
}

// Q8_0 (BlockQ8_0::from_float): one lane per 32-element block.
__global__ __launch_bounds__(256) void q8_0_append_kernel(AppendArgs a, int64_t units_per_tensor,
                                                          int nblk) {
  const int64_t unit = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (unit >= 2 * units_per_tensor) return;
  const int p = (int)(unit / units_per_tensor);
  int64_t u = unit % units_per_tensor;
  const int blk = (int)(u % nblk);
  u /= nblk;
  const int h = (int)(u % a.heads);
  u /= a.heads;
  const int b = (int)(u % a.batch);
  const int64_t t = u / a.batch;
  float x[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) x[i] = load_elem(a.src[p], a, t, b, h, blk * 32 + i);
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmax_rs(amax, __builtin_fabsf(x[i]));
  const float d = amax / 127.0f;
  const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
  uint16_t w[17];
  w[0] = f32_to_f16(d);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    uint32_t q0 = (uint8_t)rs_as_i8(__builtin_roundf(x[2 * i] * id));
    uint32_t q1 = (uint8_t)rs_as_i8(__builtin_roundf(x[2 * i + 1] * id));
    w[1 + i] = (uint16_t)(q0 | (q1 << 8));
  }
  uint16_t *dst =
      reinterpret_cast<uint16_t *>(row_ptr(a, p, t, b, h) + (int64_t)blk * 34);
#pragma unroll
  for (int i = 0; i < 17; ++i) dst[i] = w[i];
}

// F16 / BF16 rows: element-wise round-to-nearest-even conversion.
template <bool BF>
__global__ __launch_bounds__(256) void half_append_kernel(AppendArgs a, int64_t elems_per_tensor) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= 2 * elems_per_tensor) return;
  const int p = (int)(i / elems_per_tensor);
  int64_t u = i % elems_per_tensor;
  const int e = (int)(u % a.padded);
  u /= a.padded;
  const int h = (int)(u % a.heads);
  u /= a.heads;
  const int b = (int)(u % a.batch);
  const int64_t t = u / a.batch;
  const float x = load_elem(a.src[p], a, t, b, h, e);
  uint16_t *dst = reinterpret_cast<uint16_t *>(row_ptr(a, p, t, b, h));
  dst[e] = BF ? f32_to_bf16(x) : f32_to_f16(x);
}

__global__ __launch_bounds__(256) void dequant_kernel(int quant, const uint8_t *kc,
                                                      const uint8_t *vc, float *ko, float *vo,
                                                      int batch, int heads, int head_dim,
                                                      int64_t S, int64_t bpr) {
  const int64_t per = (int64_t)batch * heads * S * head_dim;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= 2 * per) return;
  const int p = (int)(i / per);
  int64_t u = i % per;  // index into [b, h, S, d]
  const int e = (int)(u % head_dim);
  u /= head_dim;
  const int64_t t = u % S;
  u /= S;
  const int h = (int)(u % heads);
  const int b = (int)(u / heads);
  const int64_t r = (t * batch + b) * heads + h;
  const uint8_t *row = (p ? vc : kc) + r * bpr;
  (p ? vo : ko)[i % per] = decode_elem(quant, row, e);
}

}  // namespace

static int launch_append_args(int quant, AppendArgs &a, hipStream_t s);

int launch_append(int quant, const float *k, const float *v, uint8_t *kc, uint8_t *vc,
                  int batch, int heads, int head_dim, int64_t n, int64_t t0, hipStream_t s) {
  if (n == 0) return PKV_OK;
  AppendArgs a;
  a.src[0] = k;
  a.src[1] = v;
  a.dst[0] = kc;
  a.dst[1] = vc;
  a.batch = batch;
  a.heads = heads;
  a.head_dim = head_dim;
  a.padded = padded_dim(quant, head_dim);
  a.n = n;
  a.t0 = t0;
  a.bpr = (int64_t)row_bytes(quant, head_dim);
  a.page_tab = nullptr;
  a.page_lg = 0;
  a.page_bytes = 0;
  a.row_mode = 0;
  return launch_append_args(quant, a, s);
}

int launch_append_paged(int quant, const float *k, const float *v, uint8_t *kpool,
                        uint8_t *vpool, const int32_t *page_tab, int page_lg,
                        int64_t page_bytes, int heads, int head_dim, int64_t n, int64_t t0,
                        hipStream_t s) {
  if (n == 0) return PKV_OK;
  AppendArgs a;
  a.src[0] = k;
  a.src[1] = v;
  a.dst[0] = kpool;
  a.dst[1] = vpool;
  a.batch = 1;
  a.heads = heads;
  a.head_dim = head_dim;
  a.padded = padded_dim(quant, head_dim);
  a.n = n;
  a.t0 = t0;
  a.bpr = (int64_t)row_bytes(quant, head_dim);
  a.page_tab = page_tab;
  a.page_lg = page_lg;
  a.page_bytes = page_bytes;
  a.row_mode = 0;
  return launch_append_args(quant, a, s);
}

int launch_append_rows(int quant, const float *k, const float *v, uint8_t *kpool, uint8_t *vpool,
                       const int64_t *row_off, int n, int heads, int head_dim, hipStream_t s) {
  if (n <= 0) return PKV_OK;
  if (n > kAppendSeqs) return set_error(PKV_ERR_ARG, "too many rows for one append launch");
  AppendArgs a;
  a.src[0] = k;
  a.src[1] = v;
  a.dst[0] = kpool;
  a.dst[1] = vpool;
  a.batch = n;
  a.heads = heads;
  a.head_dim = head_dim;
  a.padded = padded_dim(quant, head_dim);
  a.n = 1;
  a.t0 = 0;
  a.bpr = (int64_t)row_bytes(quant, head_dim);
  a.page_tab = nullptr;
  a.page_lg = 0;
  a.page_bytes = 0;
  a.row_mode = 1;
  for (int i = 0; i < n; ++i) a.row_off[i] = row_off[i];
  return launch_append_args(quant, a, s);
}

// Q4K superblocks (K and V) up to which the throughput kernel runs 4, then 2, lanes per
// sub-block (1 above)
constexpr int64_t kQ4kAppendLanes4Max = 2048, kQ4kAppendLanes2Max = 8192;

static int launch_append_args(int quant, AppendArgs &a, hipStream_t s) {
  const int batch = a.batch, heads = a.heads;
  const int64_t n = a.n;
  const int64_t rows = n * batch * heads;
  if (quant == PKV_QUANT_Q4K && rows * (a.padded / 256) * 2 <= 1024) {
    // few superblocks: latency-bound, one workgroup each
    const int nsb = a.padded / 256;
    hipLaunchKernelGGL(q4k_append_small_kernel, dim3((unsigned)(2 * rows * nsb)), dim3(256), 0,
                       s, a, nsb);
  } else if (quant == PKV_QUANT_Q4K) {
    // 8 kL lanes per superblock: split each sub-block's fit over more lanes while the
    // append has too few superblocks to give every SIMD a wave
    const int nsb = a.padded / 256;
    const int64_t units = rows * nsb;
    const int kl = 2 * units <= kQ4kAppendLanes4Max ? 4 : (2 * units <= kQ4kAppendLanes2Max ? 2 : 1);
    const int64_t threads = 2 * units * 8 * kl;
    const dim3 grid((unsigned)((threads + 255) / 256));
    if (kl == 4)
      hipLaunchKernelGGL(q4k_append_kernel<4>, grid, dim3(256), 0, s, a, units, nsb);
    else if (kl == 2)
      hipLaunchKernelGGL(q4k_append_kernel<2>, grid, dim3(256), 0, s, a, units, nsb);
    else
      hipLaunchKernelGGL(q4k_append_kernel<1>, grid, dim3(256), 0, s, a, units, nsb);
  } else if (quant == PKV_QUANT_Q8_0) {
    const int nblk = a.padded / 32;
    const int64_t units = rows * nblk;
    hipLaunchKernelGGL(q8_0_append_kernel, dim3((unsigned)((2 * units + 255) / 256)), dim3(256),
                       0, s, a, units, nblk);
  } else {
    const int64_t elems = rows * a.padded;
    if (quant == PKV_QUANT_BF16)
      hipLaunchKernelGGL(half_append_kernel<true>, dim3((unsigned)((2 * elems + 255) / 256)),
                         dim3(256), 0, s, a, elems);
    else
      hipLaunchKernelGGL(half_append_kernel<false>, dim3((unsigned)((2 * elems + 255) / 256)),
                         dim3(256), 0, s, a, elems);
  }
  PKV_HIP(hipGetLastError());
  return PKV_OK;
}

int launch_dequant(int quant, const uint8_t *kc, const uint8_t *vc, float *ko, float *vo,
                   int batch, int heads, int head_dim, int64_t S, hipStream_t s) {
  const int64_t total = 2 * (int64_t)batch * heads * S * head_dim;
  if (total == 0) return PKV_OK;
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     quant, kc, vc, ko, vo, batch, heads, head_dim, S,
                     (int64_t)row_bytes(quant, head_dim));
  PKV_HIP(hipGetLastError());
  return PKV_OK;
}

}  // namespace pkv
