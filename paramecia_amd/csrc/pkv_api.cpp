// C ABI of libpkv (include/pkv.h): cache handles, prefix snapshots and argument
// checking around the kernels. The reference behaviour each function mirrors is cited
// in include/pkv.h; error codes stand in for the reference's bail! strings.
#include <ctype.h>
#include <math.h>
#include <string.h>

#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "pkv_internal.hpp"

namespace pkv {

static thread_local std::string g_error;

int set_error(int code, const std::string &msg) {
  g_error = msg;
  return code;
}

int hip_error(hipError_t e, const char *what) {
  g_error = std::string(what) + ": " + hipGetErrorString(e);
  return PKV_ERR_HIP;
}

int Workspace::reserve(size_t need) {
  if (need <= bytes) return PKV_OK;
  if (fixed)
    return set_error(PKV_ERR_ARG, "the call needs " + std::to_string(need) +
                                      " bytes of scratch; the no-alloc scratch holds " +
                                      std::to_string(bytes));
  size_t grow = need + need / 4 + 4096;
  void *fresh = nullptr;
  PKV_HIP(hipMalloc(&fresh, grow));
  // queued kernels and captured graphs may still use the old buffer: retire it
  if (ptr) retired.push_back(ptr);
  ptr = fresh;
  bytes = grow;
  return PKV_OK;
}

int Workspace::reserve_fused(hipStream_t s) {
  if (fused) return PKV_OK;
  if (fixed) return set_error(PKV_ERR_ARG, "no in-launch combine in a no-alloc call");
  void *f = nullptr;
  PKV_HIP(hipMalloc(&f, kFusedBytes));
  const int rc = launch_zero_words(static_cast<uint32_t *>(f), kFusedBytes / 4, s);
  if (rc) {
    (void)hipFree(f);
    return rc;
  }
  fused = f;
  return PKV_OK;
}

int refuse_under_capture(hipStream_t s, const char *what) {
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  PKV_HIP(hipStreamIsCapturing(s, &cap));
  if (cap != hipStreamCaptureStatusNone)
    return set_error(PKV_ERR_UNSUPPORTED,
                     std::string(what) +
                         " allocates or clears device memory, which a captured HIP graph "
                         "cannot replay: call it before capturing");
  return PKV_OK;
}

int Workspace::reserve_host(size_t need) {
  if (fixed) return set_error(PKV_ERR_ARG, "no host staging in a no-alloc call");
  if (host_pending) {
    PKV_HIP(hipEventSynchronize(host_ev));
    host_pending = false;
  }
  if (!host_ev) PKV_HIP(hipEventCreateWithFlags(&host_ev, hipEventDisableTiming));
  if (need <= host_bytes) return PKV_OK;
  if (host) PKV_HIP(hipHostFree(host));
  host = nullptr;
  host_bytes = 0;
  PKV_HIP(hipHostMalloc(&host, need, hipHostMallocDefault));
  host_bytes = need;
  return PKV_OK;
}

int Workspace::mark_host_used(hipStream_t s) {
  PKV_HIP(hipEventRecord(host_ev, s));
  host_pending = true;
  return PKV_OK;
}

Workspace::~Workspace() {
  if (fixed) return;
  if (host_pending) (void)hipEventSynchronize(host_ev);
  if (ptr || fused || !retired.empty()) {
    (void)hipDeviceSynchronize();
    if (ptr) (void)hipFree(ptr);
    if (fused) (void)hipFree(fused);
    for (void *r : retired) (void)hipFree(r);
  }
  if (host) (void)hipHostFree(host);
  if (host_ev) (void)hipEventDestroy(host_ev);
}

static Workspace &util_workspace() {
  static thread_local Workspace ws;
  return ws;
}

static int norm_quant(int q) { return q == PKV_QUANT_NONE ? PKV_QUANT_F16 : q; }

// ---- scratch of the no-alloc entry point (pkv_flash_attn_noalloc). Each GPU the library
// runs on holds its own copy of this array until the process ends. In host code its name
// only stands for the symbol: kernels get the device address that hipGetSymbolAddress
// returns for the current device, looked up once per device and kept.
static __device__ __align__(256) unsigned char scratch[PKV_NOALLOC_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
static void *g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

static int noalloc_scratch(void **out) {
  int dev = -1;
  PKV_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return set_error(PKV_ERR_ARG, "device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_error(e, "hipGetSymbolAddress(scratch)");
    if (!p) return set_error(PKV_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PKV_OK;
}

static __device__ __align__(256) unsigned status_word;
static unsigned *g_status_ptr[kMaxDevices];

int device_status_word(unsigned **out) {
  int dev = -1;
  PKV_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return set_error(PKV_ERR_ARG, "device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_status_ptr[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(status_word));
    if (e != hipSuccess) return hip_error(e, "hipGetSymbolAddress(status_word)");
    g_status_ptr[dev] = static_cast<unsigned *>(p);
  }
  *out = g_status_ptr[dev];
  return PKV_OK;
}

}  // namespace pkv

using namespace pkv;

// ---------------------------------------------------------------- prefix object
namespace {
struct Entry {
  int kind = PKV_ENTRY_EMPTY;
  // FULL: packed rows [0, len) of K and V, exactly as stored in the cache.
  int quant = 0, batch = 0, heads = 0, head_dim = 0;
  size_t bpr = 0;
  int64_t len = 0;
  uint8_t *k = nullptr, *v = nullptr;
  // LINEAR: Gated-DeltaNet state copies.
  float *ssm = nullptr, *conv = nullptr, *gate = nullptr;
  size_t n_ssm = 0, n_conv = 0, n_gate = 0;
  // recorded on the save call's stream after the snapshot copies; a restore waits on it
  hipEvent_t ready = nullptr;
  int mark_ready(hipStream_t s) {
    if (!ready) PKV_HIP(hipEventCreateWithFlags(&ready, hipEventDisableTiming));
    PKV_HIP(hipEventRecord(ready, s));
    return PKV_OK;
  }
  void release() {
    if (ready) (void)hipEventSynchronize(ready);
    if (k) (void)hipFree(k);
    if (v) (void)hipFree(v);
    if (ssm) (void)hipFree(ssm);
    if (conv) (void)hipFree(conv);
    if (gate) (void)hipFree(gate);
    if (ready) (void)hipEventDestroy(ready);
    *this = Entry();
  }
};
}  // namespace

struct pkv_prefix {
  std::vector<uint32_t> tokens;
  std::vector<Entry> entries;
};

extern "C" {

const char *pkv_last_error(void) { return g_error.c_str(); }

int pkv_device_status(void) {
  unsigned *w = nullptr;
  int rc = device_status_word(&w);
  if (rc) return rc;
  PKV_HIP(hipDeviceSynchronize());
  unsigned v = 0;
  PKV_HIP(hipMemcpy(&v, w, sizeof v, hipMemcpyDeviceToHost));
  if (v == 0) return PKV_OK;
  const unsigned zero = 0;
  PKV_HIP(hipMemcpy(w, &zero, sizeof zero, hipMemcpyHostToDevice));
  return set_error(PKV_ERR_HIP, (v & kStatusBarrierTimeout)
                                    ? "a fused decode step's quantizer barrier timed out: its "
                                      "appended row and attention output are not valid"
                                    : "device status " + std::to_string(v));
}
const char *pkv_version(void) { return "paramecia_amd pkv 0.1 (gfx950)"; }

int pkv_quant_parse(const char *s, int *quant_out) {
  if (!s || !quant_out) return set_error(PKV_ERR_ARG, "null argument");
  std::string t(s);
  for (auto &c : t) c = (char)tolower((unsigned char)c);
  int q;
  if (t == "f16" || t == "fp16") q = PKV_QUANT_F16;
  else if (t == "bf16" || t == "bfloat16") q = PKV_QUANT_BF16;
  else if (t == "q8" || t == "q8_0") q = PKV_QUANT_Q8_0;
  else if (t == "q4" || t == "q4k" || t == "q4_k") q = PKV_QUANT_Q4K;
  else if (t == "none") q = PKV_QUANT_NONE;
  else return set_error(PKV_ERR_ARG, "unknown KV cache quantization '" + std::string(s) + "'");
  *quant_out = q;
  return PKV_OK;
}

int pkv_quant_default(void) { return PKV_QUANT_Q4K; }
int pkv_quant_block_size(int quant) { return block_size(norm_quant(quant)); }
int pkv_quant_is_ggml(int quant) { return quant == PKV_QUANT_Q8_0 || quant == PKV_QUANT_Q4K; }
size_t pkv_bytes_per_row(int quant, int head_dim) {
  return head_dim > 0 ? row_bytes(norm_quant(quant), head_dim) : 0;
}

int pkv_create(int quant, int batch, int n_kv_heads, int head_dim, int64_t max_seq_len,
               pkv_stream stream, pkv_cache **out) {
  if (!out) return set_error(PKV_ERR_ARG, "null output handle");
  *out = nullptr;
  quant = norm_quant(quant);
  if (quant < PKV_QUANT_F16 || quant > PKV_QUANT_Q4K)
    return set_error(PKV_ERR_ARG, "unknown quantization");
  if (batch <= 0 || n_kv_heads <= 0 || head_dim <= 0 || max_seq_len < 0)
    return set_error(PKV_ERR_ARG, "batch, n_kv_heads, head_dim must be > 0, max_seq_len >= 0");
  if (int rc = refuse_under_capture(static_cast<hipStream_t>(stream), "pkv_create")) return rc;
  pkv_cache *h = new pkv_cache();
  h->quant = quant;
  h->batch = batch;
  h->n_kv_heads = n_kv_heads;
  h->head_dim = head_dim;
  h->padded = padded_dim(quant, head_dim);
  h->max_seq_len = max_seq_len;
  h->seq_len = 0;
  h->bpr = row_bytes(quant, head_dim);
  h->stream = static_cast<hipStream_t>(stream);
  h->k = h->v = nullptr;
  h->order_ev = nullptr;
  const size_t total = (size_t)batch * n_kv_heads * (size_t)max_seq_len * h->bpr;
  const size_t alloc = total ? total : 256;
  hipError_t e = hipMalloc(&h->k, alloc);
  if (e == hipSuccess) e = hipMalloc(&h->v, alloc);
  if (e == hipSuccess) e = hipMemsetAsync(h->k, 0, alloc, h->stream);  // vec![0u8; total]
  if (e == hipSuccess) e = hipMemsetAsync(h->v, 0, alloc, h->stream);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&h->order_ev, hipEventDisableTiming);
  if (e != hipSuccess) {
    if (h->k) (void)hipFree(h->k);
    if (h->v) (void)hipFree(h->v);
    delete h;
    return hip_error(e, "pkv_create");
  }
  *out = h;
  return PKV_OK;
}

int pkv_destroy(pkv_cache *h) {
  if (!h) return PKV_OK;
  (void)hipStreamSynchronize(h->stream);
  (void)hipFree(h->k);
  (void)hipFree(h->v);
  if (h->order_ev) (void)hipEventDestroy(h->order_ev);
  delete h;
  return PKV_OK;
}

int pkv_set_stream(pkv_cache *h, pkv_stream stream) {
  if (!h) return set_error(PKV_ERR_ARG, "null handle");
  h->stream = static_cast<hipStream_t>(stream);
  return PKV_OK;
}

int64_t pkv_len(const pkv_cache *h) { return h ? h->seq_len : -1; }
int64_t pkv_capacity(const pkv_cache *h) { return h ? h->max_seq_len : -1; }

int pkv_geometry(const pkv_cache *h, int *quant, int *batch, int *n_kv_heads, int *head_dim,
                 size_t *bpr) {
  if (!h) return set_error(PKV_ERR_ARG, "null handle");
  if (quant) *quant = h->quant;
  if (batch) *batch = h->batch;
  if (n_kv_heads) *n_kv_heads = h->n_kv_heads;
  if (head_dim) *head_dim = h->head_dim;
  if (bpr) *bpr = h->bpr;
  return PKV_OK;
}

int pkv_truncate(pkv_cache *h, int64_t new_len) {
  if (!h) return set_error(PKV_ERR_ARG, "null handle");
  if (new_len < 0) new_len = 0;
  if (new_len < h->seq_len) h->seq_len = new_len;
  return PKV_OK;
}

int pkv_set_len(pkv_cache *h, int64_t len) {
  if (!h) return set_error(PKV_ERR_ARG, "null handle");
  if (len < 0) return set_error(PKV_ERR_ARG, "len must be >= 0");
  if (len > h->max_seq_len)
    return set_error(PKV_ERR_OVERFLOW, "Quantized KV cache overflow: trying to store " +
                                           std::to_string(len) + " tokens but max is " +
                                           std::to_string(h->max_seq_len));
  h->seq_len = len;
  return PKV_OK;
}

int pkv_clear(pkv_cache *h) {
  if (!h) return set_error(PKV_ERR_ARG, "null handle");
  h->seq_len = 0;
  return PKV_OK;
}

int pkv_resize_batch(pkv_cache *h, int batch) {
  if (!h) return set_error(PKV_ERR_ARG, "null handle");
  if (batch <= 0) return set_error(PKV_ERR_ARG, "batch must be > 0");
  if (batch == h->batch) return PKV_OK;
  if (int rc = refuse_under_capture(h->stream, "pkv_resize_batch")) return rc;
  const size_t total = (size_t)batch * h->n_kv_heads * (size_t)h->max_seq_len * h->bpr;
  const size_t alloc = total ? total : 256;
  uint8_t *k = nullptr, *v = nullptr;
  hipError_t e = hipMalloc(&k, alloc);
  if (e == hipSuccess) e = hipMalloc(&v, alloc);
  if (e == hipSuccess) e = hipMemsetAsync(k, 0, alloc, h->stream);
  if (e == hipSuccess) e = hipMemsetAsync(v, 0, alloc, h->stream);
  if (e != hipSuccess) {
    if (k) (void)hipFree(k);
    if (v) (void)hipFree(v);
    return hip_error(e, "pkv_resize_batch");
  }
  PKV_HIP(hipStreamSynchronize(h->stream));
  (void)hipFree(h->k);
  (void)hipFree(h->v);
  h->k = k;
  h->v = v;
  h->batch = batch;
  h->seq_len = 0;
  return PKV_OK;
}

// F16/BF16 caches grow instead of overflowing: the reference's float path concatenates
// every append onto the cached rows (Tensor::cat) and sets max_seq_len to the new length
// (qwen3_next.rs:2492-2516), so it has no capacity limit. Here the buffers are
// reallocated to max(need, 2 x capacity) tokens (amortised O(1) per token), rows
// [0, seq_len) copied on the handle's stream and the tail zeroed; the old buffers are
// freed once the stream has passed the copy. Not under graph capture (it allocates).
static int grow_float_cache(pkv_cache *h, int64_t need) {
  if (int rc = refuse_under_capture(h->stream, "growing an F16/BF16 cache past its capacity"))
    return rc;
  int64_t cap = h->max_seq_len * 2;
  if (cap < need) cap = need;
  const size_t row = (size_t)h->batch * h->n_kv_heads * h->bpr;  // one token's rows
  const size_t alloc = (size_t)cap * row, keep = (size_t)h->seq_len * row;
  uint8_t *k = nullptr, *v = nullptr;
  hipError_t e = hipMalloc(&k, alloc ? alloc : 256);
  if (e == hipSuccess) e = hipMalloc(&v, alloc ? alloc : 256);
  if (e == hipSuccess && keep) e = hipMemcpyAsync(k, h->k, keep, hipMemcpyDeviceToDevice, h->stream);
  if (e == hipSuccess && keep) e = hipMemcpyAsync(v, h->v, keep, hipMemcpyDeviceToDevice, h->stream);
  if (e == hipSuccess && alloc > keep) e = hipMemsetAsync(k + keep, 0, alloc - keep, h->stream);
  if (e == hipSuccess && alloc > keep) e = hipMemsetAsync(v + keep, 0, alloc - keep, h->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(h->stream);
  if (e != hipSuccess) {
    if (k) (void)hipFree(k);
    if (v) (void)hipFree(v);
    return hip_error(e, "growing an F16/BF16 cache");
  }
  (void)hipFree(h->k);
  (void)hipFree(h->v);
  h->k = k;
  h->v = v;
  h->max_seq_len = cap;
  return PKV_OK;
}

// FullAttention offset rule (qwen3_next.rs:2430-2440) then the overflow rule (:435-441);
// F16/BF16 caches grow instead (grow_float_cache).
static int position_for_append(pkv_cache *h, int64_t n, int64_t offset) {
  if (n < 0) return set_error(PKV_ERR_ARG, "n must be >= 0");
  if (offset >= 0 && offset != h->seq_len) {
    if (offset <= h->seq_len)
      h->seq_len = offset;
    else
      return set_error(PKV_ERR_OFFSET, "KV cache offset mismatch: offset=" +
                                           std::to_string(offset) + " but cache has " +
                                           std::to_string(h->seq_len) + " tokens");
  }
  if (h->seq_len + n > h->max_seq_len && !pkv_quant_is_ggml(h->quant))
    return grow_float_cache(h, h->seq_len + n);
  if (h->seq_len + n > h->max_seq_len)
    return set_error(PKV_ERR_OVERFLOW, "Quantized KV cache overflow: trying to store " +
                                           std::to_string(h->seq_len + n) +
                                           " tokens but max is " +
                                           std::to_string(h->max_seq_len));
  return PKV_OK;
}

int pkv_append(pkv_cache *h, const float *k, const float *v, int64_t n, int64_t offset) {
  if (!h || (n > 0 && (!k || !v))) return set_error(PKV_ERR_ARG, "null argument");
  int rc = position_for_append(h, n, offset);
  if (rc) return rc;
  rc = launch_append(h->quant, k, v, h->k, h->v, h->batch, h->n_kv_heads, h->head_dim, n,
                     h->seq_len, h->stream);
  if (rc) return rc;
  h->seq_len += n;
  return PKV_OK;
}

static AttnArgs cache_args(const pkv_cache *h, const float *q, int l, int num_heads, float scale,
                           int64_t seq_k, int64_t q_offset, int causal, float *out) {
  AttnArgs a;
  a.quant = h->quant;
  a.q = q;
  a.k = h->k;
  a.v = h->v;
  a.rs = h->strides();
  a.scale = scale;
  a.batch = h->batch;
  a.num_heads = num_heads;
  a.num_kv_heads = h->n_kv_heads;
  a.head_dim = h->head_dim;
  a.l = l;
  a.seq_k = seq_k;
  a.q_offset = q_offset;
  a.causal = causal;
  a.out = out;
  return a;
}

int pkv_attend(pkv_cache *h, const float *q, int l, int num_heads, float scale,
               int64_t q_offset, int causal, float *out) {
  if (!h || !q || !out) return set_error(PKV_ERR_ARG, "null argument");
  if (h->seq_len == 0) return set_error(PKV_ERR_EMPTY, "Cannot attend over an empty cache");
  return launch_attend(cache_args(h, q, l, num_heads, scale, h->seq_len, q_offset, causal, out),
                       h->ws, h->stream);
}

int pkv_append_attend(pkv_cache *h, const float *k, const float *v, const float *q,
                      int num_heads, float scale, int64_t offset, float *out) {
  if (!h || !k || !v || !q || !out) return set_error(PKV_ERR_ARG, "null argument");
  if (num_heads <= 0 || num_heads % h->n_kv_heads)
    return set_error(PKV_ERR_ARG, "num_heads must be a multiple of num_kv_heads");
  const int64_t saved = h->seq_len;
  int rc = position_for_append(h, 1, offset);
  if (rc) return rc;
  const int64_t t_new = h->seq_len;
  rc = launch_append_attend(cache_args(h, q, 1, num_heads, scale, t_new + 1, t_new, 1, out), k,
                            v, h->k, h->v, t_new, h->ws, h->stream);
  if (rc) {
    if (rc != PKV_ERR_HIP) h->seq_len = saved;
    return rc;
  }
  h->seq_len = t_new + 1;
  return PKV_OK;
}

int pkv_get_kv(pkv_cache *h, float *k_out, float *v_out) {
  if (!h) return set_error(PKV_ERR_ARG, "null handle");
  if (h->seq_len == 0) return PKV_OK;
  if (!k_out || !v_out) return set_error(PKV_ERR_ARG, "null argument");
  return launch_dequant(h->quant, h->k, h->v, k_out, v_out, h->batch, h->n_kv_heads,
                        h->head_dim, h->seq_len, h->stream);
}

int pkv_kv_storage(const pkv_cache *h, const void **k_bytes, const void **v_bytes,
                   size_t *valid_bytes, int64_t strides[4]) {
  if (!h) return set_error(PKV_ERR_ARG, "null handle");
  if (h->seq_len == 0) return set_error(PKV_ERR_EMPTY, "Cannot get storage from empty cache");
  if (k_bytes) *k_bytes = h->k;
  if (v_bytes) *v_bytes = h->v;
  if (valid_bytes) *valid_bytes = (size_t)h->seq_len * h->batch * h->n_kv_heads * h->bpr;
  if (strides) {
    const RowStrides r = h->strides();
    strides[0] = r.b;
    strides[1] = r.t;
    strides[2] = r.h;
    strides[3] = 1;
  }
  return PKV_OK;
}

static int flash_attn_ws(int quant, const float *q, const void *k_bytes, const void *v_bytes,
                         const int64_t kv_strides[3], float scale, int batch, int num_heads,
                         int num_kv_heads, int head_dim, int seq_q, int64_t seq_k,
                         int64_t q_offset, int causal, float *out, pkv_stream stream,
                         Workspace *ws) {
  quant = norm_quant(quant);
  if (!q || !k_bytes || !v_bytes || !kv_strides || !out)
    return set_error(PKV_ERR_ARG, "null argument");
  if (quant < PKV_QUANT_F16 || quant > PKV_QUANT_Q4K)
    return set_error(PKV_ERR_ARG, "unknown quantization");
  AttnArgs a;
  a.quant = quant;
  a.q = q;
  a.k = static_cast<const uint8_t *>(k_bytes);
  a.v = static_cast<const uint8_t *>(v_bytes);
  a.rs = {kv_strides[0], kv_strides[1], kv_strides[2]};
  a.scale = scale;
  a.batch = batch;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.head_dim = head_dim;
  a.l = seq_q;
  a.seq_k = seq_k;
  a.q_offset = q_offset;
  a.causal = causal;
  a.out = out;
  return launch_attend(a, ws ? *ws : util_workspace(), static_cast<hipStream_t>(stream));
}

int pkv_flash_attn(int quant, const float *q, const void *k_bytes, const void *v_bytes,
                   const int64_t kv_strides[3], float scale, int batch, int num_heads,
                   int num_kv_heads, int head_dim, int seq_q, int64_t seq_k, int64_t q_offset,
                   int causal, float *out, pkv_stream stream) {
  return flash_attn_ws(quant, q, k_bytes, v_bytes, kv_strides, scale, batch, num_heads,
                       num_kv_heads, head_dim, seq_q, seq_k, q_offset, causal, out, stream,
                       nullptr);
}

int pkv_flash_attn_noalloc(int quant, const float *q, const void *k_bytes, const void *v_bytes,
                           const int64_t kv_strides[3], float scale, int batch, int num_heads,
                           int num_kv_heads, int head_dim, int seq_q, int64_t seq_k,
                           int64_t q_offset, int causal, float *out, pkv_stream stream) {
  Workspace ws;
  ws.fixed = true;
  int rc = noalloc_scratch(&ws.ptr);
  if (rc) return rc;
  ws.bytes = PKV_NOALLOC_SCRATCH_BYTES;
  return flash_attn_ws(quant, q, k_bytes, v_bytes, kv_strides, scale, batch, num_heads,
                       num_kv_heads, head_dim, seq_q, seq_k, q_offset, causal, out, stream, &ws);
}

// ---- q/k preparation (FullAttention::forward, qwen3_next.rs:2369-2399) ----

// RotaryEmbedding::new (qwen3_next.rs:878-904): inv_freq[i] = 1f32 / (theta^(2i/n_rot) as
// f32) with the power in f64, freqs = (t as f32) * inv_freq[i] (a [max_pos, 1] x
// [1, n_rot/2] matmul: one rounded product), then f32 cos and sin (libm cosf / sinf).
int pkv_rope_tables_host(int n_rot, int64_t max_pos, double theta, float *cos_out,
                         float *sin_out) {
  if (n_rot <= 0 || (n_rot & 1) || max_pos < 0 || (max_pos > 0 && (!cos_out || !sin_out)))
    return set_error(PKV_ERR_ARG, "n_rot must be even and positive, max_pos >= 0");
  const int half = n_rot / 2;
  std::vector<float> inv(half);
  for (int i = 0; i < half; ++i)
    inv[i] = 1.0f / (float)::pow(theta, (double)(2 * i) / (double)n_rot);
  for (int64_t t = 0; t < max_pos; ++t) {
    const float ft = (float)t;
    for (int i = 0; i < half; ++i) {
      const float f = ft * inv[i];
      cos_out[t * half + i] = ::cosf(f);
      sin_out[t * half + i] = ::sinf(f);
    }
  }
  return PKV_OK;
}

int pkv_rope_create(int n_rot, int64_t max_pos, double theta, pkv_rope **out) {
  if (!out) return set_error(PKV_ERR_ARG, "null argument");
  *out = nullptr;
  if (max_pos <= 0) return set_error(PKV_ERR_ARG, "max_pos must be positive");
  if (n_rot <= 0 || (n_rot & 1)) return set_error(PKV_ERR_ARG, "n_rot must be even and positive");
  const size_t n = (size_t)max_pos * (size_t)(n_rot / 2);
  std::vector<float> c(n), sn(n);
  int rc = pkv_rope_tables_host(n_rot, max_pos, theta, c.data(), sn.data());
  if (rc) return rc;
  pkv_rope *r = new pkv_rope{n_rot, max_pos, nullptr, nullptr};
  hipError_t e = hipMalloc(&r->cos, n * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&r->sin, n * sizeof(float));
  if (e == hipSuccess) e = hipMemcpy(r->cos, c.data(), n * sizeof(float), hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(r->sin, sn.data(), n * sizeof(float), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    pkv_rope_destroy(r);
    return hip_error(e, "pkv_rope_create");
  }
  *out = r;
  return PKV_OK;
}

int pkv_rope_destroy(pkv_rope *r) {
  if (!r) return PKV_OK;
  if (r->cos) (void)hipFree(r->cos);
  if (r->sin) (void)hipFree(r->sin);
  delete r;
  return PKV_OK;
}

int pkv_rope_geometry(const pkv_rope *r, int *n_rot, int64_t *max_pos, const float **cos_tab,
                      const float **sin_tab) {
  if (!r) return set_error(PKV_ERR_ARG, "null argument");
  if (n_rot) *n_rot = r->n_rot;
  if (max_pos) *max_pos = r->max_pos;
  if (cos_tab) *cos_tab = r->cos;
  if (sin_tab) *sin_tab = r->sin;
  return PKV_OK;
}

// Checks shared by the two prepared appends; fills everything but q/q_out/k/v/t0/l.
static int prep_setup(const pkv_cache *h, const pkv_qk_prep *prep, bool with_q, int num_heads,
                      int64_t n, int64_t offset, PrepArgs &a) {
  if (!h || !prep || !prep->rope || !prep->k_alpha)
    return set_error(PKV_ERR_ARG, "null argument");
  if (with_q && (!prep->q_alpha || num_heads <= 0))
    return set_error(PKV_ERR_ARG, "q needs q_alpha and num_heads > 0");
  if (n < 0 || n >= (1ll << 31)) return set_error(PKV_ERR_ARG, "n out of range");
  const pkv_rope *r = prep->rope;
  if (r->n_rot > h->head_dim) return set_error(PKV_ERR_ARG, "n_rot exceeds head_dim");
  if (h->head_dim > 512) return set_error(PKV_ERR_UNSUPPORTED, "head_dim > 512");
  // RotaryEmbedding::apply narrows the tables at [offset, offset + n) (qwen3_next.rs:921)
  const int64_t first = offset >= 0 ? offset : h->seq_len;
  if (first + n > r->max_pos)
    return set_error(PKV_ERR_ARG, "positions " + std::to_string(first) + ".." +
                                      std::to_string(first + n) + " exceed the rope table (" +
                                      std::to_string(r->max_pos) + ")");
  a = PrepArgs{};
  a.kc = h->k;
  a.vc = h->v;
  a.q_alpha = prep->q_alpha;
  a.k_alpha = prep->k_alpha;
  a.cos_tab = r->cos;
  a.sin_tab = r->sin;
  a.eps = prep->eps;
  a.quant = h->quant;
  a.batch = h->batch;
  a.l = (int)n;
  a.num_heads = with_q ? num_heads : 0;
  a.kv_heads = h->n_kv_heads;
  a.head_dim = h->head_dim;
  a.padded = h->padded;
  a.n_rot = r->n_rot;
  a.bpr = (int64_t)h->bpr;
  a.q_rows = with_q ? (int64_t)h->batch * n * num_heads : 0;
  a.kv_rows = (int64_t)h->batch * n * h->n_kv_heads;
  return PKV_OK;
}

int pkv_append_prep(pkv_cache *h, const pkv_qk_prep *prep, const float *q, int num_heads,
                    float *q_out, const float *k, const float *v, int64_t n, int64_t offset) {
  if ((q == nullptr) != (q_out == nullptr))
    return set_error(PKV_ERR_ARG, "q and q_out go together");
  if (n > 0 && (!k || !v)) return set_error(PKV_ERR_ARG, "null argument");
  PrepArgs a;
  int rc = prep_setup(h, prep, q != nullptr, num_heads, n, offset, a);
  if (rc) return rc;
  rc = position_for_append(h, n, offset);
  if (rc) return rc;
  a.q = q;
  a.q_out = q_out;
  a.k = k;
  a.v = v;
  a.t0 = h->seq_len;
  rc = launch_prep_append(a, h->stream);
  if (rc) return rc;
  h->seq_len += n;
  return PKV_OK;
}

int pkv_append_attend_prep(pkv_cache *h, const pkv_qk_prep *prep, const float *q,
                           const float *k, const float *v, int num_heads, float scale,
                           int64_t offset, float *out) {
  if (!q || !k || !v || !out) return set_error(PKV_ERR_ARG, "null argument");
  if (h && (num_heads <= 0 || num_heads % h->n_kv_heads))
    return set_error(PKV_ERR_ARG, "num_heads must be a multiple of num_kv_heads");
  PrepArgs a;
  int rc = prep_setup(h, prep, true, num_heads, 1, offset, a);
  if (rc) return rc;
  const int64_t saved = h->seq_len;
  rc = position_for_append(h, 1, offset);
  if (rc) return rc;
  const int64_t t_new = h->seq_len;
  // Q4K at the Qwen3-Next shape: the decode kernel prepares q and the new k itself
  const DecodePrep dp{prep->q_alpha, prep->k_alpha, prep->rope->cos, prep->rope->sin,
                      prep->eps, prep->rope->n_rot};
  rc = launch_append_attend_prep_mfma(
      cache_args(h, q, 1, num_heads, scale, t_new + 1, t_new, 1, out), k, v, h->k, h->v, t_new,
      dp, h->ws, h->stream);
  if (rc == PKV_ERR_UNSUPPORTED) {
    // otherwise: the prep-append kernel (q into the handle's scratch), then attention
    rc = h->qws.reserve((size_t)h->batch * num_heads * h->head_dim * sizeof(float));
    float *qp = static_cast<float *>(h->qws.ptr);
    a.q = q;
    a.q_out = qp;
    a.k = k;
    a.v = v;
    a.t0 = t_new;
    if (!rc) rc = launch_prep_append(a, h->stream);
    if (!rc)
      rc = launch_attend(cache_args(h, qp, 1, num_heads, scale, t_new + 1, t_new, 1, out),
                         h->ws, h->stream);
  }
  if (rc) {
    if (rc != PKV_ERR_HIP) h->seq_len = saved;
    return rc;
  }
  h->seq_len = t_new + 1;
  return PKV_OK;
}

int pkv_append_attend_batched(pkv_cache *const *caches, int n, const float *k, const float *v,
                              const float *q, int num_heads, float scale, float *out,
                              pkv_stream stream) {
  if (!caches || n <= 0 || !k || !v || !q || !out) return set_error(PKV_ERR_ARG, "bad argument");
  const pkv_cache *c0 = caches[0];
  if (!c0) return set_error(PKV_ERR_ARG, "null cache");
  if (num_heads <= 0 || num_heads % c0->n_kv_heads)
    return set_error(PKV_ERR_ARG, "num_heads must be a multiple of num_kv_heads");
  std::vector<SeqDesc> seqs((size_t)n);
  for (int i = 0; i < n; ++i) {
    const pkv_cache *c = caches[i];
    if (!c || c->batch != 1 || c->quant != c0->quant || c->n_kv_heads != c0->n_kv_heads ||
        c->head_dim != c0->head_dim)
      return set_error(PKV_ERR_ARG, "batched caches must be batch-1 with equal geometry");
    if (c->seq_len + 1 > c->max_seq_len)
      return set_error(PKV_ERR_OVERFLOW, "Quantized KV cache overflow in sequence " +
                                             std::to_string(i));
    seqs[(size_t)i] = {c->k, c->v, c->seq_len + 1};
  }
  int rc = launch_append_attend_batched(c0->quant, seqs.data(), n, k, v, q, num_heads,
                                        c0->n_kv_heads, c0->head_dim, scale, out,
                                        util_workspace(), static_cast<hipStream_t>(stream));
  if (rc) return rc;
  for (int i = 0; i < n; ++i) caches[i]->seq_len += 1;
  return PKV_OK;
}

// ---------------------------------------------------------------- PrefixCache
int pkv_prefix_create(const uint32_t *tokens, size_t n_tokens, int n_layers, pkv_prefix **out) {
  if (!out || n_layers < 0 || (n_tokens && !tokens)) return set_error(PKV_ERR_ARG, "bad argument");
  pkv_prefix *p = new pkv_prefix();
  p->tokens.assign(tokens, tokens + n_tokens);
  p->entries.resize((size_t)n_layers);
  *out = p;
  return PKV_OK;
}

int pkv_prefix_free(pkv_prefix *p) {
  if (!p) return PKV_OK;
  (void)hipDeviceSynchronize();
  for (auto &e : p->entries) e.release();
  delete p;
  return PKV_OK;
}

int pkv_prefix_tokens(const pkv_prefix *p, const uint32_t **tokens, size_t *n) {
  if (!p) return set_error(PKV_ERR_ARG, "null prefix");
  if (tokens) *tokens = p->tokens.data();
  if (n) *n = p->tokens.size();
  return PKV_OK;
}

int pkv_prefix_num_layers(const pkv_prefix *p) { return p ? (int)p->entries.size() : -1; }

int pkv_prefix_entry_kind(const pkv_prefix *p, int layer) {
  if (!p || layer < 0 || layer >= (int)p->entries.size()) return -1;
  return p->entries[(size_t)layer].kind;
}

int64_t pkv_prefix_full_len(const pkv_prefix *p, int layer) {
  if (!p || layer < 0 || layer >= (int)p->entries.size()) return -1;
  const Entry &e = p->entries[(size_t)layer];
  return e.kind == PKV_ENTRY_FULL ? e.len : 0;
}

int pkv_prefix_linear_sizes(const pkv_prefix *p, int layer, size_t *n_ssm, size_t *n_conv,
                            size_t *n_gate) {
  if (!p || layer < 0 || layer >= (int)p->entries.size())
    return set_error(PKV_ERR_ARG, "bad layer");
  const Entry &e = p->entries[(size_t)layer];
  if (n_ssm) *n_ssm = e.n_ssm;
  if (n_conv) *n_conv = e.n_conv;
  if (n_gate) *n_gate = e.n_gate;
  return PKV_OK;
}

int pkv_prefix_save_full(pkv_prefix *p, int layer, const pkv_cache *h) {
  if (!p || !h || layer < 0 || layer >= (int)p->entries.size())
    return set_error(PKV_ERR_ARG, "bad argument");
  if (int rc = refuse_under_capture(h->stream, "pkv_prefix_save_full")) return rc;
  Entry &e = p->entries[(size_t)layer];
  e.release();
  if (h->seq_len == 0) return PKV_OK;  // PrefixCacheEntry::Empty
  const size_t bytes = (size_t)h->seq_len * h->batch * h->n_kv_heads * h->bpr;
  PKV_HIP(hipMalloc(&e.k, bytes));
  hipError_t er = hipMalloc(&e.v, bytes);
  if (er != hipSuccess) {
    e.release();
    return hip_error(er, "pkv_prefix_save_full");
  }
  PKV_HIP(hipMemcpyAsync(e.k, h->k, bytes, hipMemcpyDeviceToDevice, h->stream));
  PKV_HIP(hipMemcpyAsync(e.v, h->v, bytes, hipMemcpyDeviceToDevice, h->stream));
  const int rc = e.mark_ready(h->stream);
  if (rc) {
    e.release();
    return rc;
  }
  e.kind = PKV_ENTRY_FULL;
  e.quant = h->quant;
  e.batch = h->batch;
  e.heads = h->n_kv_heads;
  e.head_dim = h->head_dim;
  e.bpr = h->bpr;
  e.len = h->seq_len;
  return PKV_OK;
}

int pkv_prefix_save_linear(pkv_prefix *p, int layer, const float *ssm, size_t n_ssm,
                           const float *conv, size_t n_conv, const float *gate, size_t n_gate,
                           pkv_stream stream) {
  if (!p || layer < 0 || layer >= (int)p->entries.size() || !ssm || !conv)
    return set_error(PKV_ERR_ARG, "bad argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (int rc = refuse_under_capture(s, "pkv_prefix_save_linear")) return rc;
  Entry &e = p->entries[(size_t)layer];
  e.release();
  hipError_t er = hipMalloc(&e.ssm, (n_ssm ? n_ssm : 1) * 4);
  if (er == hipSuccess) er = hipMalloc(&e.conv, (n_conv ? n_conv : 1) * 4);
  if (er == hipSuccess) er = hipMalloc(&e.gate, (n_gate ? n_gate : 1) * 4);
  if (er == hipSuccess) er = hipMemcpyAsync(e.ssm, ssm, n_ssm * 4, hipMemcpyDeviceToDevice, s);
  if (er == hipSuccess) er = hipMemcpyAsync(e.conv, conv, n_conv * 4, hipMemcpyDeviceToDevice, s);
  if (er == hipSuccess) {
    if (gate)
      er = hipMemcpyAsync(e.gate, gate, n_gate * 4, hipMemcpyDeviceToDevice, s);
    else
      er = hipMemsetAsync(e.gate, 0, n_gate * 4, s);  // zero offset (qwen3_next.rs:4077-4093)
  }
  if (er != hipSuccess) {
    e.release();
    return hip_error(er, "pkv_prefix_save_linear");
  }
  const int rc = e.mark_ready(s);
  if (rc) {
    e.release();
    return rc;
  }
  e.kind = PKV_ENTRY_LINEAR;
  e.n_ssm = n_ssm;
  e.n_conv = n_conv;
  e.n_gate = n_gate;
  return PKV_OK;
}

// ---------------------------------------------------------------- host spill
// Blob layout (little-endian): BlobHeader, n_tokens u32 tokens, n_layers BlobEntry, then
// each entry's payload in layer order (FULL: K rows then V rows, len*batch*heads*bpr
// bytes each; LINEAR: ssm, conv, gate as f32). Everything is 8-byte aligned.
namespace {
constexpr uint32_t kBlobMagic = 0x50564B50u;  // "PKVP"
constexpr uint32_t kBlobVersion = 1;
struct BlobHeader {
  uint32_t magic, version;
  uint64_t n_tokens, n_layers, total;
};
struct BlobEntry {
  int32_t kind, quant, batch, heads, head_dim, pad;
  uint64_t bpr, len, n_ssm, n_conv, n_gate;
};
inline size_t align8(size_t x) { return (x + 7) & ~(size_t)7; }
inline size_t entry_payload(const BlobEntry &e) {
  if (e.kind == PKV_ENTRY_FULL) return 2 * align8((size_t)(e.len * (uint64_t)e.batch * e.heads * e.bpr));
  if (e.kind == PKV_ENTRY_LINEAR) return align8(e.n_ssm * 4) + align8(e.n_conv * 4) + align8(e.n_gate * 4);
  return 0;
}
BlobEntry describe(const Entry &e) {
  BlobEntry d{};
  d.kind = e.kind;
  d.quant = e.quant;
  d.batch = e.batch;
  d.heads = e.heads;
  d.head_dim = e.head_dim;
  d.bpr = e.bpr;
  d.len = (uint64_t)e.len;
  d.n_ssm = e.n_ssm;
  d.n_conv = e.n_conv;
  d.n_gate = e.n_gate;
  return d;
}
size_t blob_size(const pkv_prefix *p) {
  size_t n = sizeof(BlobHeader) + align8(p->tokens.size() * 4) + p->entries.size() * sizeof(BlobEntry);
  for (const Entry &e : p->entries) n += entry_payload(describe(e));
  return n;
}
}  // namespace

size_t pkv_prefix_serialized_size(const pkv_prefix *p) { return p ? blob_size(p) : 0; }

int pkv_prefix_serialize(const pkv_prefix *p, void *host_dst, size_t capacity, pkv_stream stream) {
  if (!p || !host_dst) return set_error(PKV_ERR_ARG, "null argument");
  const size_t total = blob_size(p);
  if (capacity < total)
    return set_error(PKV_ERR_ARG, "host buffer too small: " + std::to_string(capacity) + " < " +
                                       std::to_string(total));
  hipStream_t s = static_cast<hipStream_t>(stream);
  // the snapshot copies were issued on the caches' streams (pkv_prefix_save_full /
  // _save_linear), which need not be `stream`: a spill is rare, so wait for the device
  PKV_HIP(hipDeviceSynchronize());
  uint8_t *o = static_cast<uint8_t *>(host_dst);
  BlobHeader hd{kBlobMagic, kBlobVersion, p->tokens.size(), p->entries.size(), total};
  std::memcpy(o, &hd, sizeof hd);
  size_t at = sizeof hd;
  std::memcpy(o + at, p->tokens.data(), p->tokens.size() * 4);
  at += align8(p->tokens.size() * 4);
  for (const Entry &e : p->entries) {
    const BlobEntry d = describe(e);
    std::memcpy(o + at, &d, sizeof d);
    at += sizeof d;
  }
  for (const Entry &e : p->entries) {
    const BlobEntry d = describe(e);
    if (e.kind == PKV_ENTRY_FULL) {
      const size_t bytes = (size_t)(d.len * (uint64_t)d.batch * d.heads * d.bpr);
      PKV_HIP(hipMemcpyAsync(o + at, e.k, bytes, hipMemcpyDeviceToHost, s));
      at += align8(bytes);
      PKV_HIP(hipMemcpyAsync(o + at, e.v, bytes, hipMemcpyDeviceToHost, s));
      at += align8(bytes);
    } else if (e.kind == PKV_ENTRY_LINEAR) {
      PKV_HIP(hipMemcpyAsync(o + at, e.ssm, e.n_ssm * 4, hipMemcpyDeviceToHost, s));
      at += align8(e.n_ssm * 4);
      PKV_HIP(hipMemcpyAsync(o + at, e.conv, e.n_conv * 4, hipMemcpyDeviceToHost, s));
      at += align8(e.n_conv * 4);
      PKV_HIP(hipMemcpyAsync(o + at, e.gate, e.n_gate * 4, hipMemcpyDeviceToHost, s));
      at += align8(e.n_gate * 4);
    }
  }
  PKV_HIP(hipStreamSynchronize(s));
  return PKV_OK;
}

int pkv_prefix_deserialize(const void *host_src, size_t n, pkv_prefix **out, pkv_stream stream) {
  if (!host_src || !out) return set_error(PKV_ERR_ARG, "null argument");
  const uint8_t *in = static_cast<const uint8_t *>(host_src);
  BlobHeader hd;
  if (n < sizeof hd) return set_error(PKV_ERR_ARG, "prefix blob truncated (header)");
  std::memcpy(&hd, in, sizeof hd);
  if (hd.magic != kBlobMagic || hd.version != kBlobVersion)
    return set_error(PKV_ERR_ARG, "not a prefix blob of this version");
  if (hd.total != n || hd.n_tokens > n / 4 || hd.n_layers > n / sizeof(BlobEntry))
    return set_error(PKV_ERR_ARG, "prefix blob size mismatch");
  size_t at = sizeof hd + align8(hd.n_tokens * 4);
  const size_t table = at;
  if (at + hd.n_layers * sizeof(BlobEntry) > n) return set_error(PKV_ERR_ARG, "prefix blob truncated");
  std::vector<BlobEntry> ds(hd.n_layers);
  size_t payload = 0;
  for (size_t i = 0; i < hd.n_layers; ++i) {
    std::memcpy(&ds[i], in + table + i * sizeof(BlobEntry), sizeof(BlobEntry));
    const BlobEntry &d = ds[i];
    if (d.kind == PKV_ENTRY_FULL) {
      // every factor bounded before the product: len * batch * heads * bpr <= n
      if (d.batch <= 0 || d.heads <= 0 || d.head_dim <= 0 || d.bpr == 0 || d.bpr > (1u << 20) ||
          (uint64_t)d.batch * d.heads > (1ull << 20) || d.bpr != row_bytes(d.quant, d.head_dim) ||
          d.len > n / ((uint64_t)d.batch * d.heads * d.bpr))
        return set_error(PKV_ERR_ARG, "prefix blob: bad full-attention entry " + std::to_string(i));
    } else if (d.kind == PKV_ENTRY_LINEAR) {
      if (d.n_ssm > n || d.n_conv > n || d.n_gate > n)
        return set_error(PKV_ERR_ARG, "prefix blob: bad linear entry " + std::to_string(i));
    } else if (d.kind != PKV_ENTRY_EMPTY) {
      return set_error(PKV_ERR_ARG, "prefix blob: unknown entry kind");
    }
    payload += entry_payload(d);
    if (payload > n) return set_error(PKV_ERR_ARG, "prefix blob truncated (payload)");
  }
  at += hd.n_layers * sizeof(BlobEntry);
  if (at + payload != n) return set_error(PKV_ERR_ARG, "prefix blob size mismatch (payload)");
  hipStream_t s = static_cast<hipStream_t>(stream);
  pkv_prefix *p = new pkv_prefix();
  p->tokens.resize(hd.n_tokens);
  std::memcpy(p->tokens.data(), in + sizeof hd, hd.n_tokens * 4);
  p->entries.resize(hd.n_layers);
  auto fail = [&](hipError_t er) {
    (void)hipStreamSynchronize(s);
    for (auto &e : p->entries) e.release();
    delete p;
    return hip_error(er, "pkv_prefix_deserialize");
  };
  for (size_t i = 0; i < hd.n_layers; ++i) {
    const BlobEntry &d = ds[i];
    Entry &e = p->entries[i];
    hipError_t er = hipSuccess;
    if (d.kind == PKV_ENTRY_FULL) {
      const size_t bytes = (size_t)(d.len * (uint64_t)d.batch * d.heads * d.bpr);
      er = hipMalloc(&e.k, bytes ? bytes : 1);
      if (er == hipSuccess) er = hipMalloc(&e.v, bytes ? bytes : 1);
      if (er == hipSuccess) er = hipMemcpyAsync(e.k, in + at, bytes, hipMemcpyHostToDevice, s);
      at += align8(bytes);
      if (er == hipSuccess) er = hipMemcpyAsync(e.v, in + at, bytes, hipMemcpyHostToDevice, s);
      at += align8(bytes);
      e.quant = d.quant;
      e.batch = d.batch;
      e.heads = d.heads;
      e.head_dim = d.head_dim;
      e.bpr = d.bpr;
      e.len = (int64_t)d.len;
    } else if (d.kind == PKV_ENTRY_LINEAR) {
      er = hipMalloc(&e.ssm, (d.n_ssm ? d.n_ssm : 1) * 4);
      if (er == hipSuccess) er = hipMalloc(&e.conv, (d.n_conv ? d.n_conv : 1) * 4);
      if (er == hipSuccess) er = hipMalloc(&e.gate, (d.n_gate ? d.n_gate : 1) * 4);
      if (er == hipSuccess) er = hipMemcpyAsync(e.ssm, in + at, d.n_ssm * 4, hipMemcpyHostToDevice, s);
      at += align8(d.n_ssm * 4);
      if (er == hipSuccess) er = hipMemcpyAsync(e.conv, in + at, d.n_conv * 4, hipMemcpyHostToDevice, s);
      at += align8(d.n_conv * 4);
      if (er == hipSuccess) er = hipMemcpyAsync(e.gate, in + at, d.n_gate * 4, hipMemcpyHostToDevice, s);
      at += align8(d.n_gate * 4);
      e.n_ssm = d.n_ssm;
      e.n_conv = d.n_conv;
      e.n_gate = d.n_gate;
    }
    e.kind = d.kind;
    if (er != hipSuccess) return fail(er);
  }
  const hipError_t er = hipStreamSynchronize(s);
  if (er != hipSuccess) return fail(er);
  *out = p;
  return PKV_OK;
}

int pkv_prefix_restore(const pkv_prefix *p, const pkv_layer_target *targets, int n_layers,
                       int mode, size_t *n_tokens_out, pkv_stream stream) {
  if (!p || (n_layers && !targets)) return set_error(PKV_ERR_ARG, "bad argument");
  if ((size_t)n_layers != p->entries.size())
    return set_error(PKV_ERR_LAYERS, "Prefix cache layer count mismatch: " +
                                         std::to_string(p->entries.size()) + " vs " +
                                         std::to_string(n_layers));
  if (mode != PKV_RESTORE_BYTES && mode != PKV_RESTORE_REQUANTIZE)
    return set_error(PKV_ERR_ARG, "unknown restore mode");
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Validate every layer before writing anything.
  for (int i = 0; i < n_layers; ++i) {
    const Entry &e = p->entries[(size_t)i];
    const pkv_layer_target &t = targets[i];
    if (t.cache && (t.ssm || t.conv || t.gate_offset))
      return set_error(PKV_ERR_ARG, "layer " + std::to_string(i) + ": both cache and state set");
    if (t.cache && e.kind == PKV_ENTRY_FULL) {
      const pkv_cache *c = t.cache;
      if (c->quant != e.quant || c->n_kv_heads != e.heads || c->head_dim != e.head_dim ||
          c->batch != e.batch)
        return set_error(PKV_ERR_LAYOUT, "layer " + std::to_string(i) +
                                             ": snapshot geometry differs from the cache");
      if (e.len > c->max_seq_len)
        return set_error(PKV_ERR_OVERFLOW, "Quantized KV cache overflow: trying to store " +
                                               std::to_string(e.len) + " tokens but max is " +
                                               std::to_string(c->max_seq_len));
    }
    if (!t.cache && e.kind == PKV_ENTRY_LINEAR) {
      if (!t.ssm || !t.conv || !t.gate_offset)
        return set_error(PKV_ERR_ARG, "layer " + std::to_string(i) + ": missing state targets");
      if (e.n_ssm > t.ssm_cap || e.n_conv > t.conv_cap || e.n_gate > t.gate_cap)
        return set_error(PKV_ERR_LAYOUT, "layer " + std::to_string(i) +
                                             ": saved state (" + std::to_string(e.n_ssm) + ", " +
                                             std::to_string(e.n_conv) + ", " +
                                             std::to_string(e.n_gate) +
                                             " floats) exceeds the restore targets");
    }
  }
  // Order the launch after the snapshot copies and after work already queued on the
  // target caches' streams (an attention still reading rows about to be overwritten).
  // Under stream capture there is no cross-stream ordering to add: an event recorded
  // outside the capture cannot be waited on inside it, and a cache stream made to wait on
  // the capturing stream would join the capture unjoined. The graph's own order applies
  // when it is replayed.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  PKV_HIP(hipStreamIsCapturing(s, &cap));
  const bool capturing = cap != hipStreamCaptureStatusNone;
  for (int i = 0; i < n_layers && !capturing; ++i) {
    const Entry &e = p->entries[(size_t)i];
    const pkv_layer_target &t = targets[i];
    const bool used = t.cache ? e.kind == PKV_ENTRY_FULL : e.kind == PKV_ENTRY_LINEAR;
    if (used && e.ready) PKV_HIP(hipStreamWaitEvent(s, e.ready, 0));
    if (t.cache && t.cache->stream != s) {
      PKV_HIP(hipEventRecord(t.cache->order_ev, t.cache->stream));
      PKV_HIP(hipStreamWaitEvent(s, t.cache->order_ev, 0));
    }
  }
  std::vector<void *> dst;
  std::vector<const void *> src;
  std::vector<size_t> bytes;
  for (int i = 0; i < n_layers; ++i) {
    const Entry &e = p->entries[(size_t)i];
    const pkv_layer_target &t = targets[i];
    if (t.cache) {
      if (e.kind == PKV_ENTRY_FULL) {
        if (mode == PKV_RESTORE_BYTES) {
          const size_t nb = (size_t)e.len * e.batch * e.heads * e.bpr;
          dst.push_back(t.cache->k); src.push_back(e.k); bytes.push_back(nb);
          dst.push_back(t.cache->v); src.push_back(e.v); bytes.push_back(nb);
        }
      }
    } else if (e.kind == PKV_ENTRY_LINEAR) {
      dst.push_back(t.ssm); src.push_back(e.ssm); bytes.push_back(e.n_ssm * 4);
      dst.push_back(t.conv); src.push_back(e.conv); bytes.push_back(e.n_conv * 4);
      dst.push_back(t.gate_offset); src.push_back(e.gate); bytes.push_back(e.n_gate * 4);
    }
  }
  int rc = launch_copy_segments(dst.data(), src.data(), bytes.data(), (int)dst.size(),
                                util_workspace(), s);
  if (rc) return rc;
  int rc_order = PKV_OK;  // the caches' streams wait for everything below
  auto order_caches = [&]() {
    for (int i = 0; i < n_layers && !rc_order && !capturing; ++i) {
      pkv_cache *c = targets[i].cache;
      if (!c || c->stream == s) continue;
      hipError_t er = hipEventRecord(c->order_ev, s);
      if (er == hipSuccess) er = hipStreamWaitEvent(c->stream, c->order_ev, 0);
      if (er != hipSuccess) rc_order = hip_error(er, "pkv_prefix_restore (stream order)");
    }
    return rc_order;
  };
  for (int i = 0; i < n_layers; ++i) {
    const Entry &e = p->entries[(size_t)i];
    const pkv_layer_target &t = targets[i];
    if (t.cache) {
      pkv_cache *c = t.cache;
      if (e.kind != PKV_ENTRY_FULL) {
        c->seq_len = 0;  // Empty / wrong kind -> clear_kv_cache (qwen3_next.rs:2874-2882)
        continue;
      }
      if (mode == PKV_RESTORE_REQUANTIZE) {
        // clear(); append(dequantized saved K/V) — the reference's restore path.
        const size_t n = (size_t)e.batch * e.heads * (size_t)e.len * e.head_dim;
        rc = c->ws.reserve(2 * n * sizeof(float));
        if (rc) return rc;
        float *kf = static_cast<float *>(c->ws.ptr), *vf = kf + n;
        rc = launch_dequant(e.quant, e.k, e.v, kf, vf, e.batch, e.heads, e.head_dim, e.len, s);
        if (!rc)
          rc = launch_append(c->quant, kf, vf, c->k, c->v, c->batch, c->n_kv_heads,
                             c->head_dim, e.len, 0, s);
        if (rc) {
          order_caches();
          return rc;
        }
      }
      c->seq_len = e.len;
    } else if (t.state_valid) {
      *t.state_valid = e.kind == PKV_ENTRY_LINEAR ? 1 : 0;
    }
  }
  if (order_caches()) return rc_order;
  if (n_tokens_out) *n_tokens_out = p->tokens.size();
  return PKV_OK;
}

int pkv_deltanet_step(const float *q, const float *k, const float *v, const float *gate,
                      const float *beta, float *state, float *gate_offset, float *out,
                      int batch, int heads, int head_dim, float scale, float eps,
                      pkv_stream stream) {
  if (!q || !k || !v || !gate || !beta || !state || !out)
    return set_error(PKV_ERR_ARG, "null argument");
  if (batch <= 0 || heads <= 0 || head_dim <= 0)
    return set_error(PKV_ERR_ARG, "batch, heads and head_dim must be > 0");
  return launch_deltanet_step(q, k, v, gate, beta, state, gate_offset, out, batch, heads,
                              head_dim, scale, eps, static_cast<hipStream_t>(stream));
}

// From this many tokens on, the k-quant projection runs as the batched MFMA form (each
// decoded weight serves 32 tokens); below it, per-token GEMV workgroups.
constexpr int kOprojMfmaMinBatch = 8;

int pkv_gated_oproj(const float *attn, const float *gate, const void *w, int w_type, float *out,
                    int batch, int in_dim, int out_dim, pkv_stream stream) {
  if (!attn || !w || !out) return set_error(PKV_ERR_ARG, "null argument");
  if (batch <= 0 || in_dim <= 0 || out_dim <= 0)
    return set_error(PKV_ERR_ARG, "batch, in_dim and out_dim must be > 0");
  const auto *wb = static_cast<const uint8_t *>(w);
  const auto s = static_cast<hipStream_t>(stream);
  if (batch >= kOprojMfmaMinBatch &&
      (w_type == PKV_WTYPE_Q4K || w_type == PKV_WTYPE_Q5K || w_type == PKV_WTYPE_Q6K))
    return launch_oproj_mfma(attn, gate, wb, w_type, out, batch, in_dim, out_dim,
                             util_workspace(), s);
  return launch_oproj(attn, gate, wb, w_type, out, batch, in_dim, out_dim, s);
}

int pkv_gated_oproj_q4k(const float *attn, const float *gate, const void *w_q4k, float *out,
                        int batch, int in_dim, int out_dim, pkv_stream stream) {
  return pkv_gated_oproj(attn, gate, w_q4k, PKV_WTYPE_Q4K, out, batch, in_dim, out_dim, stream);
}

int pkv_fill_normal(float *dst, size_t n, uint64_t seed, uint64_t stream_id, float scale,
                    pkv_stream stream) {
  if (!dst && n) return set_error(PKV_ERR_ARG, "null destination");
  return launch_fill_normal(dst, n, seed, stream_id, scale, static_cast<hipStream_t>(stream));
}

int pkv_scale_channels(float *x, size_t rows, int dim, const int *channels, int n_ch,
                       float factor, pkv_stream stream) {
  if (!x || (n_ch && !channels) || dim <= 0) return set_error(PKV_ERR_ARG, "bad argument");
  return launch_scale_channels(x, rows, dim, channels, n_ch, factor,
                               static_cast<hipStream_t>(stream));
}

int pkv_copy_segments(void *const *dst, const void *const *src, const size_t *bytes, int n,
                      pkv_stream stream) {
  if (n < 0 || (n && (!dst || !src || !bytes))) return set_error(PKV_ERR_ARG, "bad argument");
  return launch_copy_segments(dst, src, bytes, n, util_workspace(),
                              static_cast<hipStream_t>(stream));
}

}  // extern "C"
