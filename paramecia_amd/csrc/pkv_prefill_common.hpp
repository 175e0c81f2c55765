// Shared parts of the MFMA prefill-chunk kernels (Q4K and Q8_0 caches, the Qwen3-Next
// full-attention shape: 16 query heads, 2 KV heads, head_dim 256): the kernel arguments,
// the work plan (16 query positions x one KV head x one key split per workgroup, splits
// chosen to fill about 256 workgroups) and the kernel that merges the key splits' (m, l,
// o) partials. Include-only; every symbol has internal linkage.
//
// Partial layout: part[batch * nsplit + split][kv head][pos * 8 + head of the group][258]:
// entries 0-255 in tile order (entry i holds element tile_e(i / 16, i % 16)), then the
// row's running max m (log2 units) and sum l.
#pragma once
#include "pkv_decode_split.hpp"

namespace pkv {
namespace {

constexpr int kPfWaves = 8;
constexpr int kPfThreads = 64 * kPfWaves;
constexpr int kPosPerWG = 16;  // query positions per workgroup, two per wave
constexpr int kRaw = 3;        // raw block stages in flight
constexpr int kPfTargetWGs = 256;
constexpr float kPfLazy = 8.0f;
constexpr int kMaxMergeSplits = 16;

struct PrefillArgs {
  const float *q;  // [B][l][16][256]
  const uint8_t *k, *v;
  int64_t rs_b, rs_t, rs_h;
  int64_t seq_k;     // keys in the cache
  int64_t q_offset;  // query i sees key j iff !causal || j <= i + q_offset
  int l, causal;
  int ntiles, nsplit, bps;  // position tiles, key splits, blocks per split
  int ngroups;              // (batch, split, KV head) groups: 2 * nsplit * batch
  float sl2;                // scale * log2(e)
  float *part;  // [B * nsplit][2][l * 8][258] partials in tile order (nsplit > 1)
  float *out;   // [B][l][16][256] (nsplit == 1)
};

// A workgroup's tile, KV head, key split and batch row in the 1-D grid of ntiles *
// ngroups workgroups: consecutive workgroups take consecutive (batch, split, KV head)
// groups. The dispatcher deals workgroups to the 8 XCDs round-robin, so with 8 groups
// (the 512-token chunk: 2 KV heads x 4 splits) every workgroup that streams one group's
// key range runs on one XCD and the range is fetched into that XCD's L2 once, not by all
// eight.
struct PfWork {
  int tile, kvg, split, b;
};
__device__ __forceinline__ PfWork prefill_work(const PrefillArgs &a) {
  const int L = blockIdx.x, grp = L % a.ngroups, z = grp >> 1;
  return PfWork{L / a.ngroups, grp & 1, z % a.nsplit, z / a.nsplit};
}

// Merge the key splits: out[b][pos][8 kvg + hh][e] = sum_s o_s 2^(m_s - M) / sum_s l_s 2^(m_s - M).
// One workgroup of 256 threads per 8 rows and batch: 32 threads per row, each taking 8
// consecutive tile-order entries; every split's (m, l) and entries are loaded before any
// is used (nsplit <= kMaxMergeSplits).
__global__ __launch_bounds__(256) void prefill_merge_kernel(const float *part, int nsplit,
                                                                int l, float *out) {
  const int r8 = threadIdx.x >> 5, j = threadIdx.x & 31;
  const int row = blockIdx.x * 8 + r8, b = blockIdx.y;  // row = kvg * l * 8 + pos * 8 + hh
  if (row >= 2 * l * 8) return;
  const int kvg = row / (l * 8), rr = row % (l * 8), pos = rr >> 3, hh = rr & 7;
  const int64_t split_stride = (int64_t)2 * l * 8 * 258;
  const float *base = part + (((int64_t)(b * nsplit) * 2 + kvg) * l * 8 + rr) * 258;
  float2 ml[kMaxMergeSplits], v[kMaxMergeSplits][4];
#pragma unroll
  for (int s = 0; s < kMaxMergeSplits; ++s) {
    if (s < nsplit) {
      const float *pr = base + s * split_stride;
      ml[s] = *reinterpret_cast<const float2 *>(pr + 256);
#pragma unroll
      for (int k = 0; k < 4; ++k) v[s][k] = *reinterpret_cast<const float2 *>(pr + 8 * j + 2 * k);
    }
  }
  float M = -INFINITY;
#pragma unroll
  for (int s = 0; s < kMaxMergeSplits; ++s)
    if (s < nsplit) M = fmaxf(M, ml[s].x);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, L = 0.0f;
#pragma unroll
  for (int s = 0; s < kMaxMergeSplits; ++s) {
    if (s < nsplit) {
      const float f = (ml[s].x == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(ml[s].x - M);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc[2 * k] += f * v[s][k].x;
        acc[2 * k + 1] += f * v[s][k].y;
      }
      L += f * ml[s].y;
    }
  }
  float *orow = out + (((int64_t)b * l + pos) * 16 + 8 * kvg + hh) * 256;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int idx = 8 * j + k;
    orow[tile_e(idx >> 4, idx & 15)] = L > 0.0f ? acc[k] / L : 0.0f;
  }
}

}  // namespace

// The plan of a prefill chunk over 32-key blocks: position tiles, key splits (enough
// workgroups to fill the GPU, at most kMaxMergeSplits), the partials' workspace.
static inline int prefill_plan(const AttnArgs &a, float sl2, Workspace &ws, PrefillArgs &d) {
  d.q = a.q;
  d.k = a.k;
  d.v = a.v;
  d.rs_b = a.rs.b;
  d.rs_t = a.rs.t;
  d.rs_h = a.rs.h;
  d.seq_k = a.seq_k;
  d.q_offset = a.q_offset;
  d.l = a.l;
  d.causal = a.causal ? 1 : 0;
  d.sl2 = sl2;
  d.ntiles = (a.l + kPosPerWG - 1) / kPosPerWG;
  const int nblk = (int)((a.seq_k + 31) / 32);
  const int base = d.ntiles * 2 * a.batch;
  int nsplit = (kPfTargetWGs + base - 1) / base;
  if (nsplit > kMaxMergeSplits) nsplit = kMaxMergeSplits;
  if (nsplit > nblk) nsplit = nblk > 0 ? nblk : 1;
  if (nsplit < 1) nsplit = 1;
  d.bps = (nblk + nsplit - 1) / nsplit;
  if (d.bps < 1) d.bps = 1;
  d.nsplit = nsplit;
  d.ngroups = 2 * nsplit * a.batch;
  d.out = a.out;
  d.part = nullptr;
  if (nsplit > 1) {
    const size_t need = (size_t)a.batch * nsplit * 2 * a.l * 8 * 258 * sizeof(float);
    const int rc = ws.reserve(need);
    if (rc) return rc;
    d.part = static_cast<float *>(ws.ptr);
  }
  return PKV_OK;
}

// The split merge after a prefill kernel that wrote partials (nsplit > 1).
static inline int prefill_merge(const PrefillArgs &d, int batch, hipStream_t s) {
  if (d.nsplit <= 1) return PKV_OK;
  hipLaunchKernelGGL(prefill_merge_kernel, dim3((unsigned)((2 * d.l * 8 + 7) / 8), (unsigned)batch),
                     dim3(256), 0, s, d.part, d.nsplit, d.l, d.out);
  PKV_HIP(hipGetLastError());
  return PKV_OK;
}

}  // namespace pkv
