// Paged KV caches for multi-sequence serving: a pool of fixed-size pages for one layer,
// sequences as page lists with reference-counted sharing. The reference preallocates one
// PreallocatedQuantizedKvCache per layer and sequence at max_seq_len
// (paramecia-model/src/qwen3_next.rs:343-643), and its one serving caller keeps a single
// sequence whose prefix cache is a deep copy (paramecia-llm/src/backend/local.rs:743-800,
// qwen3_next.rs:856-864); a pool instead holds many sequences of any lengths, and a
// prefix entry shared by several requests is one set of pages.
//
// Layout: plane K and plane V, each n_pages x page_bytes; page p holds the rows of
// page_tokens tokens x n_kv_heads (row (t, h) at p * page_bytes + (t * H + h) * bpr), the
// rows of a batch-1 cache of capacity page_tokens in the same encoding. Rows are written
// only by the quantize-on-append kernels; the planes start zeroed, so every row decodes
// to finite values.
//
// Sharing: fork copies a sequence's page list and raises each page's count. A page is
// written only while its count is 1: appending into a shared, partly filled last page
// first copies its rows into a fresh page (copy on write). Pages return to the free list
// when their count drops to 0.
//
// Attention: the decode step of the model's shape (Q4K / Q8_0, 16 query heads, 2 KV
// heads, head_dim 256, one query that sees every key) runs the split-K decode kernels
// with one segment per page (launch_paged_decode_*): no copy. Other calls (prefill
// chunks, other shapes and encodings, get_kv) first gather the sequence's rows into a
// contiguous scratch with one copy launch, then run the contiguous-cache kernels; for a
// prefill chunk the copy is small beside the attention itself.
#include <cstring>
#include <string>
#include <vector>

#include "pkv_internal.hpp"

struct pkv_pool {
  int quant, n_kv_heads, head_dim;
  int page_tokens, page_lg, n_pages;
  size_t bpr, page_bytes;
  uint8_t *k, *v;
  hipStream_t stream;
  std::vector<int32_t> free_list;  // page ids, taken from the back
  std::vector<int32_t> refs;       // sequences holding each page
  int live_seqs;
  pkv::Workspace ws;      // split-K partials, copy tables, pinned staging
  pkv::Workspace gather;  // contiguous rows of one sequence
  // Pinned staging slots for segment and page tables, used in turn: a slot is reused only
  // after the copy that read it has run (its event), which for kStages slots is kStages
  // calls back, so the host rarely waits for the device
  static constexpr int kStages = 8;
  void *stage[kStages] = {};
  size_t stage_bytes[kStages] = {};
  hipEvent_t stage_ev[kStages] = {};
  bool stage_pending[kStages] = {};
  int stage_next = 0;
};

struct pkv_seq {
  pkv_pool *pool;
  std::vector<int32_t> pages;  // in token order
  int64_t len;
  int32_t *d_pages;  // device copy of `pages` (append and decode kernels), n_pages entries
  bool d_stale = true;  // `pages` changed since d_pages was last written
};

namespace pkv {
namespace {

int take_page(pkv_pool *p) {
  const int32_t id = p->free_list.back();
  p->free_list.pop_back();
  p->refs[(size_t)id] = 1;
  return id;
}

void release_page(pkv_pool *p, int32_t id) {
  if (--p->refs[(size_t)id] == 0) p->free_list.push_back(id);
}

// pages [keep, end) of s go back to the pool
void release_tail(pkv_seq *s, size_t keep) {
  while (s->pages.size() > keep) {
    release_page(s->pool, s->pages.back());
    s->pages.pop_back();
    s->d_stale = true;
  }
}

size_t pages_for(const pkv_pool *p, int64_t tokens) {
  return (size_t)((tokens + p->page_tokens - 1) >> p->page_lg);
}

uint8_t *page_k(const pkv_pool *p, int32_t id) { return p->k + (size_t)id * p->page_bytes; }
uint8_t *page_v(const pkv_pool *p, int32_t id) { return p->v + (size_t)id * p->page_bytes; }

// A free pinned staging slot of at least `bytes` (waits for the copy that last read it).
int stage_acquire(pkv_pool *p, size_t bytes, int *slot) {
  const int i = p->stage_next;
  p->stage_next = (i + 1) % pkv_pool::kStages;
  if (p->stage_pending[i]) {
    PKV_HIP(hipEventSynchronize(p->stage_ev[i]));
    p->stage_pending[i] = false;
  }
  if (p->stage_bytes[i] < bytes) {  // (sized at creation for every page of the pool)
    if (p->stage[i]) PKV_HIP(hipHostFree(p->stage[i]));
    p->stage[i] = nullptr;
    p->stage_bytes[i] = 0;
    const size_t want = bytes < 4096 ? 4096 : bytes + bytes / 2;
    PKV_HIP(hipHostMalloc(&p->stage[i], want, hipHostMallocDefault));
    p->stage_bytes[i] = want;
  }
  *slot = i;
  return PKV_OK;
}

// The slot's copy is queued: mark it in use until the stream passes this point.
int stage_release(pkv_pool *p, int slot) {
  PKV_HIP(hipEventRecord(p->stage_ev[slot], p->stream));
  p->stage_pending[slot] = true;
  return PKV_OK;
}

// The page table of s into its device copy, staged through a pinned slot.
// Bring d_pages up to date (a copy only when the page list changed since the last one).
// The copy reads a pinned staging slot, so it cannot be captured in a HIP graph.
int sync_pages(pkv_seq *s) {
  pkv_pool *p = s->pool;
  const size_t bytes = s->pages.size() * sizeof(int32_t);
  if (!s->d_stale || bytes == 0) return PKV_OK;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  PKV_HIP(hipStreamIsCapturing(p->stream, &cap));
  if (cap != hipStreamCaptureStatusNone)
    return set_error(PKV_ERR_UNSUPPORTED,
                     "a paged sequence whose page list changed cannot be captured in a graph");
  int slot = 0;
  int rc = stage_acquire(p, bytes, &slot);
  if (rc) return rc;
  memcpy(p->stage[slot], s->pages.data(), bytes);
  PKV_HIP(hipMemcpyAsync(s->d_pages, p->stage[slot], bytes, hipMemcpyHostToDevice, p->stream));
  rc = stage_release(p, slot);
  if (rc) return rc;
  s->d_stale = false;
  return PKV_OK;
}

// The rows of tokens [0, len) of s, contiguous ([token][head] rows) in p->gather: K at
// *kc, V at *vc.
int gather_rows(const pkv_seq *s, uint8_t **kc, uint8_t **vc) {
  pkv_pool *p = s->pool;
  const size_t row = (size_t)p->n_kv_heads * p->bpr;
  const size_t plane = (size_t)s->len * row;
  int rc = p->gather.reserve(2 * plane + 256);
  if (rc) return rc;
  uint8_t *base = static_cast<uint8_t *>(p->gather.ptr);
  *kc = base;
  *vc = base + plane;
  std::vector<void *> dst;
  std::vector<const void *> src;
  std::vector<size_t> bytes;
  for (size_t j = 0; j < s->pages.size(); ++j) {
    const int64_t t0 = (int64_t)j << p->page_lg;
    const int64_t n = s->len - t0 < p->page_tokens ? s->len - t0 : p->page_tokens;
    if (n <= 0) break;
    for (int pl = 0; pl < 2; ++pl) {
      dst.push_back((pl ? *vc : *kc) + (size_t)t0 * row);
      src.push_back(pl ? page_v(p, s->pages[j]) : page_k(p, s->pages[j]));
      bytes.push_back((size_t)n * row);
    }
  }
  return launch_copy_segments(dst.data(), src.data(), bytes.data(), (int)dst.size(), p->ws,
                              p->stream);
}

// What n more tokens of s need: `cow` when the page holding token len is shared and
// partly filled (its rows are first copied into a page of s's own), `fresh` pages taken
// from the pool in all (the copy's page included). Safe for any page list length.
struct RoomPlan {
  bool cow;
  size_t fresh;
};
RoomPlan plan_room(const pkv_seq *s, int64_t n) {
  const pkv_pool *p = s->pool;
  const size_t have = s->pages.size(), need = pages_for(p, s->len + n);
  const size_t cur = (size_t)(s->len >> p->page_lg);  // the page that holds token len
  const bool cow = n > 0 && (s->len & (p->page_tokens - 1)) != 0 && cur < have &&
                   p->refs[(size_t)s->pages[cur]] > 1;
  return RoomPlan{cow, (need > have ? need - have : 0) + (cow ? 1 : 0)};
}

// A page list that changes (a copy on write, new pages) or that the device copy does not
// yet hold must be copied to the device from pinned memory (sync_pages), which a HIP graph
// cannot replay: refused under capture, before anything changes.
int capture_guard(const pkv_seq *s, int64_t n) {
  if (!s->d_stale && plan_room(s, n).fresh == 0) return PKV_OK;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  PKV_HIP(hipStreamIsCapturing(s->pool->stream, &cap));
  if (cap != hipStreamCaptureStatusNone)
    return set_error(PKV_ERR_UNSUPPORTED,
                     "a paged sequence whose page list changes cannot be captured in a graph");
  return PKV_OK;
}

// The state make_room changed, to put back when a later step of the same call fails.
struct RoomUndo {
  size_t size = 0;      // page list length before
  size_t cow_idx = 0;   // the copied page's index
  int32_t cow_old = -1; // the shared page it replaced (-1: no copy on write)
  int32_t cow_new = -1;
};

// Pages for n more tokens of s: a shared, partly filled page is first copied into a page
// of s's own, then fresh pages follow. PKV_ERR_OVERFLOW, with nothing changed, when the
// pool lacks them (`reserved`: pages already promised to other sequences of the call; a
// non-null `reserved` only counts). `undo` (optional) records the change for undo_room.
int make_room(pkv_seq *s, int64_t n, size_t *reserved, RoomUndo *undo = nullptr) {
  pkv_pool *p = s->pool;
  const RoomPlan plan = plan_room(s, n);
  const size_t need = pages_for(p, s->len + n);
  const size_t avail = p->free_list.size() - (reserved ? *reserved : 0);
  if (plan.fresh > avail)
    return set_error(PKV_ERR_OVERFLOW, "Paged KV pool overflow: " + std::to_string(plan.fresh) +
                                           " more pages needed, " + std::to_string(avail) +
                                           " free");
  if (reserved) {  // a dry run: count only
    *reserved += plan.fresh;
    return PKV_OK;
  }
  if (undo) *undo = RoomUndo{s->pages.size(), 0, -1, -1};
  if (plan.cow) {
    // the shared, partly filled page: its rows into a page of this sequence's own
    const size_t idx = (size_t)(s->len >> p->page_lg);
    const int32_t old = s->pages[idx], mine = take_page(p);
    const size_t bytes = (size_t)(s->len & (p->page_tokens - 1)) * p->n_kv_heads * p->bpr;
    hipError_t e = hipMemcpyAsync(page_k(p, mine), page_k(p, old), bytes,
                                  hipMemcpyDeviceToDevice, p->stream);
    if (e == hipSuccess)
      e = hipMemcpyAsync(page_v(p, mine), page_v(p, old), bytes, hipMemcpyDeviceToDevice,
                         p->stream);
    if (e != hipSuccess) {
      release_page(p, mine);
      return hip_error(e, "copy on write of a shared page");
    }
    release_page(p, old);
    s->pages[idx] = mine;
    s->d_stale = true;
    if (undo) {
      undo->cow_idx = idx;
      undo->cow_old = old;
      undo->cow_new = mine;
    }
  }
  while (s->pages.size() < need) {
    s->pages.push_back(take_page(p));
    s->d_stale = true;
  }
  return PKV_OK;
}

// Put s's page list back as it was before make_room (a later step of the call failed):
// the pages it took return to the pool and a copied page gives way to the shared one
// again. The device copy of the list may already hold the new one: it is marked stale.
void undo_room(pkv_seq *s, const RoomUndo &u) {
  pkv_pool *p = s->pool;
  while (s->pages.size() > u.size) {
    release_page(p, s->pages.back());
    s->pages.pop_back();
  }
  if (u.cow_new >= 0) {
    ++p->refs[(size_t)u.cow_old];
    s->pages[u.cow_idx] = u.cow_old;
    release_page(p, u.cow_new);
  }
  s->d_stale = true;
}

bool fast_decode_shape(const pkv_pool *p, int num_heads) {
  return (p->quant == PKV_QUANT_Q4K || p->quant == PKV_QUANT_Q8_0) && p->head_dim == 256 &&
         p->n_kv_heads == 2 && num_heads == 16;
}

// Paged decode of seqs[0..n) (n <= kMaxPagedSeqs, all in pool p, each non-empty), query
// row i of q for sequence i. With k non-null (a fused step; Q4K pools): each sequence
// holds len keys (possibly none) and a page for one more token; the decode launch also
// quantizes k / v ([n][n_kv_heads][head_dim]) into row len of each sequence and attends
// to it, so sequence i sees len + 1 keys (the caller then advances len).
int paged_decode(pkv_pool *p, pkv_seq *const *seqs, int n, const float *q, float scale,
                 float *out, const float *k = nullptr, const float *v = nullptr) {
  if (p->quant == PKV_QUANT_Q4K) {
    PagedSeqDesc d[kMaxPagedSeqs];
    for (int i = 0; i < n; ++i) {
      const int rc = sync_pages(seqs[i]);
      if (rc) return rc;
      d[i] = PagedSeqDesc{seqs[i]->d_pages, seqs[i]->len};
    }
    const PagedPoolDesc pd{p->k, p->v, (int64_t)p->page_bytes, p->page_lg};
    return launch_paged_decode_q4k(d, n, pd, q, out, scale, p->ws, p->stream, k, v);
  }
  std::vector<PagedSeg> segs;
  for (int i = 0; i < n; ++i) {
    const pkv_seq *s = seqs[i];
    for (size_t j = 0; j < pages_for(p, s->len); ++j) {
      const int64_t t0 = (int64_t)j << p->page_lg;
      const int64_t m = s->len - t0 < p->page_tokens ? s->len - t0 : p->page_tokens;
      segs.push_back(PagedSeg{page_k(p, s->pages[j]), page_v(p, s->pages[j]), m, i});
    }
  }
  const int64_t rs_t = (int64_t)p->n_kv_heads * (int64_t)p->bpr, rs_h = (int64_t)p->bpr;
  int slot = -1;
  void *stage = nullptr;
  if (segs.size() > (size_t)kPagedArgSegs) {  // a device table, staged through a pinned slot
    const int rc = stage_acquire(p, segs.size() * kPagedSegBytes, &slot);
    if (rc) return rc;
    stage = p->stage[slot];
  }
  const int rc = launch_paged_decode_q8(segs.data(), (int)segs.size(), n, p->page_tokens, q, out,
                                        rs_t, rs_h, scale, stage, p->ws, p->stream);
  if (slot >= 0) {
    const int rs = stage_release(p, slot);
    if (!rc && rs) return rs;
  }
  return rc;
}

}  // namespace
}  // namespace pkv

using namespace pkv;

int pkv_pool_create(int quant, int n_kv_heads, int head_dim, int page_tokens, int n_pages,
                    pkv_stream stream, pkv_pool **out) {
  if (!out) return set_error(PKV_ERR_ARG, "null output handle");
  *out = nullptr;
  if (quant == PKV_QUANT_NONE) quant = PKV_QUANT_F16;
  if (quant < PKV_QUANT_F16 || quant > PKV_QUANT_Q4K)
    return set_error(PKV_ERR_ARG, "unknown quantization");
  if (n_kv_heads <= 0 || head_dim <= 0 || n_pages <= 0)
    return set_error(PKV_ERR_ARG, "n_kv_heads, head_dim and n_pages must be > 0");
  if (page_tokens < 32 || page_tokens > (1 << 20) || (page_tokens & (page_tokens - 1)) != 0)
    return set_error(PKV_ERR_ARG, "page_tokens must be a power of two in [32, 2^20]");
  if (int rc = refuse_under_capture(static_cast<hipStream_t>(stream), "pkv_pool_create"))
    return rc;
  pkv_pool *p = new pkv_pool();
  p->quant = quant;
  p->n_kv_heads = n_kv_heads;
  p->head_dim = head_dim;
  p->page_tokens = page_tokens;
  p->page_lg = 0;
  while ((1 << p->page_lg) < page_tokens) ++p->page_lg;
  p->n_pages = n_pages;
  p->bpr = row_bytes(quant, head_dim);
  p->page_bytes = (size_t)page_tokens * n_kv_heads * p->bpr;
  p->stream = static_cast<hipStream_t>(stream);
  p->k = p->v = nullptr;
  p->live_seqs = 0;
  const size_t plane = (size_t)n_pages * p->page_bytes;
  hipError_t e = hipMalloc(&p->k, plane);
  if (e == hipSuccess) e = hipMalloc(&p->v, plane);
  if (e == hipSuccess) e = hipMemsetAsync(p->k, 0, plane, p->stream);
  if (e == hipSuccess) e = hipMemsetAsync(p->v, 0, plane, p->stream);
  if (e != hipSuccess) {
    if (p->k) (void)hipFree(p->k);
    if (p->v) (void)hipFree(p->v);
    delete p;
    return set_error(PKV_ERR_HIP, std::string("pool allocation: ") + hipGetErrorString(e));
  }
  // the staging slots up front (pinned allocations can wait for the device): each holds a
  // segment table of every page of the pool, or a page table
  const size_t stage_bytes = (size_t)n_pages * kPagedSegBytes + 4096;
  for (int i = 0; i < pkv_pool::kStages && e == hipSuccess; ++i) {
    e = hipHostMalloc(&p->stage[i], stage_bytes, hipHostMallocDefault);
    if (e == hipSuccess) p->stage_bytes[i] = stage_bytes;
    if (e == hipSuccess) e = hipEventCreateWithFlags(&p->stage_ev[i], hipEventDisableTiming);
  }
  if (e != hipSuccess) {
    for (int i = 0; i < pkv_pool::kStages; ++i) {
      if (p->stage[i]) (void)hipHostFree(p->stage[i]);
      if (p->stage_ev[i]) (void)hipEventDestroy(p->stage_ev[i]);
    }
    (void)hipFree(p->k);
    (void)hipFree(p->v);
    delete p;
    return set_error(PKV_ERR_HIP, std::string("pool staging allocation: ") + hipGetErrorString(e));
  }
  p->refs.assign((size_t)n_pages, 0);
  p->free_list.reserve((size_t)n_pages);
  for (int i = n_pages - 1; i >= 0; --i) p->free_list.push_back(i);  // page 0 first
  *out = p;
  return PKV_OK;
}

int pkv_pool_destroy(pkv_pool *p) {
  if (!p) return PKV_OK;
  if (p->live_seqs != 0)
    return set_error(PKV_ERR_ARG, "the pool still has " + std::to_string(p->live_seqs) +
                                      " sequences");
  PKV_HIP(hipStreamSynchronize(p->stream));
  (void)hipFree(p->k);
  (void)hipFree(p->v);
  for (int i = 0; i < pkv_pool::kStages; ++i) {
    if (p->stage[i]) (void)hipHostFree(p->stage[i]);
    if (p->stage_ev[i]) (void)hipEventDestroy(p->stage_ev[i]);
  }
  delete p;
  return PKV_OK;
}

int pkv_pool_free_pages(const pkv_pool *p) { return p ? (int)p->free_list.size() : -1; }

int pkv_pool_set_stream(pkv_pool *p, pkv_stream stream) {
  if (!p) return set_error(PKV_ERR_ARG, "null handle");
  p->stream = static_cast<hipStream_t>(stream);
  return PKV_OK;
}

int pkv_seq_create(pkv_pool *p, pkv_seq **out) {
  if (!p || !out) return set_error(PKV_ERR_ARG, "null argument");
  *out = nullptr;
  pkv_seq *s = new pkv_seq();
  s->pool = p;
  s->len = 0;
  s->d_pages = nullptr;
  const hipError_t e = hipMalloc(&s->d_pages, (size_t)p->n_pages * sizeof(int32_t));
  if (e != hipSuccess) {
    delete s;
    return set_error(PKV_ERR_HIP, std::string("page table allocation: ") + hipGetErrorString(e));
  }
  ++p->live_seqs;
  *out = s;
  return PKV_OK;
}

int pkv_seq_destroy(pkv_seq *s) {
  if (!s) return PKV_OK;
  // work queued on the pool's stream may still read this sequence's pages and table
  PKV_HIP(hipStreamSynchronize(s->pool->stream));
  release_tail(s, 0);
  (void)hipFree(s->d_pages);
  --s->pool->live_seqs;
  delete s;
  return PKV_OK;
}

int64_t pkv_seq_len(const pkv_seq *s) { return s ? s->len : -1; }

int pkv_seq_pages(const pkv_seq *s) { return s ? (int)s->pages.size() : -1; }

int pkv_seq_fork(const pkv_seq *s, pkv_seq **out) {
  if (!s || !out) return set_error(PKV_ERR_ARG, "null argument");
  pkv_seq *c = nullptr;
  int rc = pkv_seq_create(s->pool, &c);
  if (rc) return rc;
  c->pages = s->pages;
  c->len = s->len;
  for (int32_t id : c->pages) ++s->pool->refs[(size_t)id];
  *out = c;
  return PKV_OK;
}

int pkv_seq_truncate(pkv_seq *s, int64_t new_len) {
  if (!s) return set_error(PKV_ERR_ARG, "null handle");
  if (new_len < 0) new_len = 0;
  if (new_len < s->len) {
    s->len = new_len;
    release_tail(s, pages_for(s->pool, new_len));
  }
  return PKV_OK;
}

int pkv_seq_append(pkv_seq *s, const float *k, const float *v, int64_t n, int64_t offset) {
  if (!s || (n > 0 && (!k || !v))) return set_error(PKV_ERR_ARG, "null argument");
  if (n < 0) return set_error(PKV_ERR_ARG, "n must be >= 0");
  pkv_pool *p = s->pool;
  // the cache offset rule (qn:2430-2440): a smaller offset rewinds, a larger one fails
  if (offset >= 0 && offset != s->len) {
    if (offset > s->len)
      return set_error(PKV_ERR_OFFSET, "KV cache offset mismatch: offset=" +
                                           std::to_string(offset) + " but cache has " +
                                           std::to_string(s->len) + " tokens");
    pkv_seq_truncate(s, offset);
  }
  if (n == 0) return PKV_OK;
  int rc = capture_guard(s, n);
  if (rc) return rc;
  RoomUndo undo;
  rc = make_room(s, n, nullptr, &undo);
  if (rc) return rc;
  rc = sync_pages(s);
  if (!rc)
    rc = launch_append_paged(p->quant, k, v, p->k, p->v, s->d_pages, p->page_lg,
                             (int64_t)p->page_bytes, p->n_kv_heads, p->head_dim, n, s->len,
                             p->stream);
  if (rc) {
    undo_room(s, undo);
    return rc;
  }
  s->len += n;
  return PKV_OK;
}

int pkv_seq_append_batched(pkv_seq *const *seqs, int n, const float *k, const float *v) {
  if (!seqs || n <= 0 || !k || !v) return set_error(PKV_ERR_ARG, "null argument or n <= 0");
  pkv_pool *p = seqs[0] ? seqs[0]->pool : nullptr;
  for (int i = 0; i < n; ++i) {
    if (!seqs[i] || seqs[i]->pool != p)
      return set_error(PKV_ERR_ARG, "every sequence must belong to the same pool");
    for (int j = 0; j < i; ++j)
      if (seqs[j] == seqs[i]) return set_error(PKV_ERR_ARG, "a sequence appears twice");
  }
  // all or nothing: count the pages first
  size_t reserved = 0;
  for (int i = 0; i < n; ++i) {
    const int rc = make_room(seqs[i], 1, &reserved);
    if (rc) return rc;
  }
  const size_t per = (size_t)p->n_kv_heads * p->head_dim;
  for (int i0 = 0; i0 < n; i0 += kAppendSeqs) {
    const int m = n - i0 < kAppendSeqs ? n - i0 : kAppendSeqs;
    int64_t off[kAppendSeqs];
    RoomUndo undo[kAppendSeqs];
    int made = 0, rc = PKV_OK;
    for (; made < m; ++made) {
      pkv_seq *s = seqs[i0 + made];
      rc = make_room(s, 1, nullptr, &undo[made]);
      if (rc) break;
      const int64_t t = s->len;
      off[made] = (int64_t)s->pages[(size_t)(t >> p->page_lg)] * (int64_t)p->page_bytes +
                  (t & (p->page_tokens - 1)) * (int64_t)p->n_kv_heads * (int64_t)p->bpr;
    }
    if (!rc)
      rc = launch_append_rows(p->quant, k + i0 * per, v + i0 * per, p->k, p->v, off, m,
                              p->n_kv_heads, p->head_dim, p->stream);
    if (rc) {  // this chunk queued nothing: its page lists go back (earlier chunks stay)
      for (int i = made - 1; i >= 0; --i) undo_room(seqs[i0 + i], undo[i]);
      return rc;
    }
    for (int i = 0; i < m; ++i) ++seqs[i0 + i]->len;
  }
  return PKV_OK;
}

int pkv_seq_attend(pkv_seq *s, const float *q, int l, int num_heads, float scale,
                   int64_t q_offset, int causal, float *out) {
  if (!s || !q || !out) return set_error(PKV_ERR_ARG, "null argument");
  if (s->len == 0) return set_error(PKV_ERR_EMPTY, "Cannot attend over an empty cache");
  pkv_pool *p = s->pool;
  if (l <= 0 || num_heads <= 0 || num_heads % p->n_kv_heads)
    return set_error(PKV_ERR_ARG, "l > 0 and num_heads a multiple of num_kv_heads");
  if (l == 1 && fast_decode_shape(p, num_heads) && (!causal || q_offset + 1 >= s->len)) {
    pkv_seq *one[1] = {s};
    return paged_decode(p, one, 1, q, scale, out);
  }
  uint8_t *kc = nullptr, *vc = nullptr;
  int rc = gather_rows(s, &kc, &vc);
  if (rc) return rc;
  AttnArgs a;
  a.quant = p->quant;
  a.q = q;
  a.k = kc;
  a.v = vc;
  a.rs = RowStrides{(int64_t)s->len * p->n_kv_heads * (int64_t)p->bpr,
                    (int64_t)p->n_kv_heads * (int64_t)p->bpr, (int64_t)p->bpr};
  a.scale = scale;
  a.batch = 1;
  a.num_heads = num_heads;
  a.num_kv_heads = p->n_kv_heads;
  a.head_dim = p->head_dim;
  a.l = l;
  a.seq_k = s->len;
  a.q_offset = q_offset;
  a.causal = causal;
  a.out = out;
  return launch_attend(a, p->ws, p->stream);
}

int pkv_seq_decode_batched(pkv_seq *const *seqs, int n, const float *q, int num_heads,
                           float scale, float *out) {
  if (!seqs || n <= 0 || !q || !out) return set_error(PKV_ERR_ARG, "null argument or n <= 0");
  pkv_pool *p = seqs[0] ? seqs[0]->pool : nullptr;
  for (int i = 0; i < n; ++i) {
    if (!seqs[i] || seqs[i]->pool != p)
      return set_error(PKV_ERR_ARG, "every sequence must belong to the same pool");
    if (seqs[i]->len == 0)
      return set_error(PKV_ERR_EMPTY, "Cannot attend over an empty cache");
  }
  if (num_heads <= 0 || num_heads % p->n_kv_heads)
    return set_error(PKV_ERR_ARG, "num_heads must be a multiple of num_kv_heads");
  const size_t qrow = (size_t)num_heads * p->head_dim;
  if (!fast_decode_shape(p, num_heads)) {
    for (int i = 0; i < n; ++i) {
      const int rc = pkv_seq_attend(seqs[i], q + i * qrow, 1, num_heads, scale, seqs[i]->len - 1,
                                    1, out + i * qrow);
      if (rc) return rc;
    }
    return PKV_OK;
  }
  for (int i0 = 0; i0 < n; i0 += kMaxPagedSeqs) {
    const int m = n - i0 < kMaxPagedSeqs ? n - i0 : kMaxPagedSeqs;
    const int rc = paged_decode(p, seqs + i0, m, q + i0 * qrow, scale, out + i0 * qrow);
    if (rc) return rc;
  }
  return PKV_OK;
}

int pkv_seq_append_decode_batched(pkv_seq *const *seqs, int n, const float *k, const float *v,
                                  const float *q, int num_heads, float scale, float *out) {
  if (!seqs || n <= 0 || !k || !v || !q || !out)
    return set_error(PKV_ERR_ARG, "null argument or n <= 0");
  pkv_pool *p = seqs[0] ? seqs[0]->pool : nullptr;
  for (int i = 0; i < n; ++i) {
    if (!seqs[i] || seqs[i]->pool != p)
      return set_error(PKV_ERR_ARG, "every sequence must belong to the same pool");
    for (int j = 0; j < i; ++j)
      if (seqs[j] == seqs[i]) return set_error(PKV_ERR_ARG, "a sequence appears twice");
  }
  if (num_heads <= 0 || num_heads % p->n_kv_heads)
    return set_error(PKV_ERR_ARG, "num_heads must be a multiple of num_kv_heads");
  if (p->quant != PKV_QUANT_Q4K || !fast_decode_shape(p, num_heads)) {
    const int rc = pkv_seq_append_batched(seqs, n, k, v);
    if (rc) return rc;
    return pkv_seq_decode_batched(seqs, n, q, num_heads, scale, out);
  }
  // all or nothing for every refusal: the pages are counted and the capture status
  // checked for every sequence before any chunk changes a page list or queues work
  size_t reserved = 0;
  for (int i = 0; i < n; ++i) {
    int rc = make_room(seqs[i], 1, &reserved);
    if (!rc) rc = capture_guard(seqs[i], 1);
    if (rc) return rc;
  }
  const size_t per = (size_t)p->n_kv_heads * p->head_dim, qrow = (size_t)num_heads * p->head_dim;
  for (int i0 = 0; i0 < n; i0 += kMaxPagedSeqs) {
    const int m = n - i0 < kMaxPagedSeqs ? n - i0 : kMaxPagedSeqs;
    RoomUndo undo[kMaxPagedSeqs];
    int made = 0, rc = PKV_OK;
    for (; made < m && !rc; ++made) rc = make_room(seqs[i0 + made], 1, nullptr, &undo[made]);
    if (rc) --made;  // the failed one changed nothing
    if (!rc)
      rc = paged_decode(p, seqs + i0, m, q + i0 * qrow, scale, out + i0 * qrow, k + i0 * per,
                        v + i0 * per);
    if (rc) {  // nothing of this chunk was queued: its page lists go back as they were
      for (int i = made - 1; i >= 0; --i) undo_room(seqs[i0 + i], undo[i]);
      return rc;
    }
    for (int i = 0; i < m; ++i) ++seqs[i0 + i]->len;
  }
  return PKV_OK;
}

int pkv_seq_get_kv(const pkv_seq *s, float *k_out, float *v_out) {
  if (!s) return set_error(PKV_ERR_ARG, "null handle");
  if (s->len == 0) return PKV_OK;
  if (!k_out || !v_out) return set_error(PKV_ERR_ARG, "null argument");
  uint8_t *kc = nullptr, *vc = nullptr;
  int rc = gather_rows(s, &kc, &vc);
  if (rc) return rc;
  const pkv_pool *p = s->pool;
  return launch_dequant(p->quant, kc, vc, k_out, v_out, 1, p->n_kv_heads, p->head_dim, s->len,
                        p->stream);
}
