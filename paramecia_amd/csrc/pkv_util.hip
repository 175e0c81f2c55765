// Utility kernels: seeded synthetic data, channel scaling, and the batched
// gather/copy used by PrefixCache restore (qwen3_next.rs:2819-2884 restores every
// layer separately on the CPU; here all segments of a prefix go out in one launch).
#include <string.h>

#include <vector>

#include "pkv_internal.hpp"
#include "pkv_scalar.hpp"

namespace pkv {
namespace {

__global__ __launch_bounds__(256) void fill_normal_kernel(float *dst, size_t n, uint64_t seed,
                                                          uint64_t stream_id, float scale) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    dst[i] = seeded_normal(seed, stream_id, i) * scale;
}

constexpr int kMaxChannels = 64;
struct Channels {
  int ch[kMaxChannels];
};

__global__ __launch_bounds__(256) void scale_channels_kernel(float *x, size_t rows, int dim,
                                                             Channels c, int n_ch,
                                                             float factor) {
  const size_t total = rows * (size_t)n_ch;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t r = i / n_ch;
    x[r * dim + c.ch[i % n_ch]] *= factor;
  }
}

// Segment table for the batched copy. Chunk c of the launch belongs to the segment s
// with first_chunk[s] <= c < first_chunk[s+1].
struct Segment {
  uint8_t *dst;
  const uint8_t *src;
  uint64_t bytes;
  uint64_t first_chunk;
};
// 16 KB per chunk: one round of four 16-byte loads per lane of a 256-lane workgroup.
// Small chunks and nontemporal loads and stores measured fastest for large HBM copies
// here (6.5 TB/s read + write, against 5.3-5.9 TB/s for 64-256 KB chunks or cached
// accesses, and 5.3 TB/s for hipMemcpyAsync).
constexpr uint64_t kChunk = 16 * 1024;
// One workgroup per chunk (the hardware dispatcher keeps every CU fed; a persistent grid
// of 2048 workgroups walking the chunks measured 7% slower on a 532 MB restore). Larger
// copies loop: workgroup wg takes chunks wg, wg + grid, ...
constexpr int kCopyWGs = 1 << 20;

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// The segment table reaches the kernel in one of two forms: as a kernel argument when it
// holds at most kArgSegs segments (no host-to-device copy, nothing to wait for: a
// prefix restore of a 48-layer model has 132 segments), otherwise as a device array.
constexpr int kArgSegs = 136;
struct ArgTable {
  uint8_t *dst[kArgSegs];
  const uint8_t *src[kArgSegs];
  uint64_t bytes[kArgSegs];
  uint32_t first[kArgSegs];
  __device__ uint64_t first_chunk(int i) const { return first[i]; }
  __device__ Segment get(int i) const { return Segment{dst[i], src[i], bytes[i], first[i]}; }
};
struct DevTable {
  const Segment *segs;
  __device__ uint64_t first_chunk(int i) const { return segs[i].first_chunk; }
  __device__ Segment get(int i) const { return segs[i]; }
};
static_assert(sizeof(ArgTable) + 16 <= 4096, "kernel arguments");

template <typename Table>
__global__ __launch_bounds__(256) void copy_segments_kernel(Table tab, int n, uint64_t chunks) {
  for (uint64_t c = blockIdx.x; c < chunks; c += gridDim.x) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {  // last segment with first_chunk <= c
      const int mid = (lo + hi + 1) >> 1;
      if (tab.first_chunk(mid) <= c) lo = mid; else hi = mid - 1;
    }
    const Segment sg = tab.get(lo);
    const uint64_t off = (c - sg.first_chunk) * kChunk;
    const uint64_t len = sg.bytes - off < kChunk ? sg.bytes - off : kChunk;
    uint8_t *d = sg.dst + off;
    const uint8_t *s = sg.src + off;
    const bool aligned = ((reinterpret_cast<uintptr_t>(d) | reinterpret_cast<uintptr_t>(s)) & 15) == 0;
    uint64_t done = 0;
    if (aligned) {
      const uint64_t n16 = len / 16;
      const v4u *s4 = reinterpret_cast<const v4u *>(s);
      v4u *d4 = reinterpret_cast<v4u *>(d);
      v4u v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint64_t i = threadIdx.x + 256 * u;
        if (i < n16) v[u] = __builtin_nontemporal_load(s4 + i);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint64_t i = threadIdx.x + 256 * u;
        if (i < n16) __builtin_nontemporal_store(v[u], d4 + i);
      }
      done = n16 * 16;
    }
    for (uint64_t i = done + threadIdx.x; i < len; i += 256) d[i] = s[i];
  }
}

__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t *dst, size_t n) {
  for (size_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) dst[i] = 0u;
}

}  // namespace

int launch_zero_words(uint32_t *dst, size_t n, hipStream_t s) {
  if (n == 0) return PKV_OK;
  size_t blocks = (n + 255) / 256;
  if (blocks > 1024) blocks = 1024;
  hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)blocks), dim3(256), 0, s, dst, n);
  PKV_HIP(hipGetLastError());
  return PKV_OK;
}

int launch_fill_normal(float *dst, size_t n, uint64_t seed, uint64_t stream_id, float scale,
                       hipStream_t s) {
  if (n == 0) return PKV_OK;
  size_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(fill_normal_kernel, dim3((unsigned)blocks), dim3(256), 0, s, dst, n, seed,
                     stream_id, scale);
  PKV_HIP(hipGetLastError());
  return PKV_OK;
}

int launch_scale_channels(float *x, size_t rows, int dim, const int *ch, int n_ch, float factor,
                          hipStream_t s) {
  if (n_ch < 0 || n_ch > kMaxChannels) return set_error(PKV_ERR_ARG, "at most 64 channels");
  Channels c{};
  for (int i = 0; i < n_ch; ++i) {
    if (ch[i] < 0 || ch[i] >= dim) return set_error(PKV_ERR_ARG, "channel index out of range");
    c.ch[i] = ch[i];
  }
  const size_t total = rows * (size_t)n_ch;
  if (total == 0) return PKV_OK;
  size_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(scale_channels_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, rows,
                     dim, c, n_ch, factor);
  PKV_HIP(hipGetLastError());
  return PKV_OK;
}

int launch_copy_segments(void *const *dst, const void *const *src, const size_t *bytes, int n,
                         Workspace &ws, hipStream_t s) {
  std::vector<Segment> segs;
  uint64_t chunks = 0;
  for (int i = 0; i < n; ++i) {
    if (bytes[i] == 0) continue;
    Segment g;
    g.dst = static_cast<uint8_t *>(dst[i]);
    g.src = static_cast<const uint8_t *>(src[i]);
    g.bytes = bytes[i];
    g.first_chunk = chunks;
    chunks += (bytes[i] + kChunk - 1) / kChunk;
    segs.push_back(g);
  }
  if (segs.empty()) return PKV_OK;
  const unsigned grid = (unsigned)(chunks < (uint64_t)kCopyWGs ? chunks : (uint64_t)kCopyWGs);
  const int ns = (int)segs.size();
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  PKV_HIP(hipStreamIsCapturing(s, &cap));
  if (cap != hipStreamCaptureStatusNone && (ns > kArgSegs || chunks >= (1ull << 32))) {
    // Under stream capture the table travels in kernel arguments only, kArgSegs segments
    // per launch: a table copied from the pinned host buffer would be read when the graph
    // is replayed, after later calls have reused the buffer.
    for (int i0 = 0; i0 < ns; i0 += kArgSegs) {
      const int m = ns - i0 < kArgSegs ? ns - i0 : kArgSegs;
      ArgTable t;
      uint64_t c = 0;
      for (int i = 0; i < m; ++i) {
        const Segment &g = segs[(size_t)(i0 + i)];
        t.dst[i] = g.dst;
        t.src[i] = g.src;
        t.bytes[i] = g.bytes;
        t.first[i] = (uint32_t)c;
        c += (g.bytes + kChunk - 1) / kChunk;
      }
      if (c >= (1ull << 32)) return set_error(PKV_ERR_UNSUPPORTED, "copy of 2^32 chunks or more");
      const unsigned gm = (unsigned)(c < (uint64_t)kCopyWGs ? c : (uint64_t)kCopyWGs);
      hipLaunchKernelGGL(copy_segments_kernel<ArgTable>, dim3(gm), dim3(256), 0, s, t, m, c);
      PKV_HIP(hipGetLastError());
    }
    return PKV_OK;
  }
  if (ns <= kArgSegs && chunks < (1ull << 32)) {
    ArgTable t;
    for (int i = 0; i < ns; ++i) {
      t.dst[i] = segs[i].dst;
      t.src[i] = segs[i].src;
      t.bytes[i] = segs[i].bytes;
      t.first[i] = (uint32_t)segs[i].first_chunk;
    }
    hipLaunchKernelGGL(copy_segments_kernel<ArgTable>, dim3(grid), dim3(256), 0, s, t, ns,
                       chunks);
  } else {
    const size_t table = segs.size() * sizeof(Segment);
    int rc = ws.reserve(table);
    if (!rc) rc = ws.reserve_host(table);
    if (rc) return rc;
    memcpy(ws.host, segs.data(), table);
    PKV_HIP(hipMemcpyAsync(ws.ptr, ws.host, table, hipMemcpyHostToDevice, s));
    rc = ws.mark_host_used(s);
    if (rc) return rc;
    hipLaunchKernelGGL(copy_segments_kernel<DevTable>, dim3(grid), dim3(256), 0, s,
                       DevTable{static_cast<const Segment *>(ws.ptr)}, ns, chunks);
  }
  PKV_HIP(hipGetLastError());
  return PKV_OK;
}

}  // namespace pkv
