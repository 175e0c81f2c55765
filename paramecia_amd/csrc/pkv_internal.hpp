// Internal declarations shared by the libpkv translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/pkv.h"

namespace pkv {

// Thread-local error slot behind pkv_last_error().
int set_error(int code, const std::string &msg);
int hip_error(hipError_t e, const char *what);

#define PKV_HIP(call)                                     \
  do {                                                    \
    hipError_t e_ = (call);                               \
    if (e_ != hipSuccess) return ::pkv::hip_error(e_, #call); \
  } while (0)

inline int block_size(int quant) {
  return quant == PKV_QUANT_Q8_0 ? 32 : quant == PKV_QUANT_Q4K ? 256 : 1;
}
inline int padded_dim(int quant, int head_dim) {
  int bs = block_size(quant);
  return (head_dim + bs - 1) / bs * bs;
}
inline size_t row_bytes(int quant, int head_dim) {
  int p = padded_dim(quant, head_dim);
  switch (quant) {
    case PKV_QUANT_Q8_0: return (size_t)(p / 32) * 34;
    case PKV_QUANT_Q4K: return (size_t)(p / 256) * 144;
    case PKV_QUANT_F16:
    case PKV_QUANT_BF16: return (size_t)p * 2;
    default: return 0;
  }
}

// Device status word of the current device (a static __device__ word, one per GPU): kernels
// that give up a bounded wait set a bit with an atomic OR; pkv_device_status() reads and
// clears it.
constexpr unsigned kStatusBarrierTimeout = 1u;  // the fused quantizer's barrier of waves 0-3
int device_status_word(unsigned **out);

// PKV_ERR_UNSUPPORTED when `s` is capturing a HIP graph: for calls that allocate device
// memory or clear it with hipMemsetAsync, neither of which a replay can repeat.
int refuse_under_capture(hipStream_t s, const char *what);

// Byte addressing of packed rows: row(b, t, h) = base + b*sb + t*st + h*sh.
struct RowStrides {
  int64_t b, t, h;
};

// Split-K scratch owned by a cache handle or by a stateless call.
// Device scratch grows (hipMalloc) on demand, never inside a kernel. A buffer it grows
// out of is retired, not freed: a HIP graph captured earlier keeps its address in its
// kernel arguments and writes there on every replay, so retired buffers live until the
// workspace is destroyed (growth is geometric: they add up to less than 4x the last
// size). The pinned host buffer stages small descriptor tables; an event guards its
// reuse. A fixed workspace (fixed = true) wraps caller-provided device memory: reserve()
// never allocates and refuses a need beyond `bytes` (PKV_ERR_ARG); nothing is freed.
struct Workspace {
  void *ptr = nullptr;
  size_t bytes = 0;
  bool fixed = false;
  std::vector<void *> retired;
  void *host = nullptr;
  size_t host_bytes = 0;
  hipEvent_t host_ev = nullptr;
  bool host_pending = false;
  // The partials and control words of one-row decodes whose combine runs inside the
  // decode launch: kFusedSlots split-K partials ([slot][16][256] floats, then
  // [slot][16] (m, l) pairs) and kFusedWords words, zeroed by a kernel on the stream when
  // first allocated. Every launch leaves them in a state the next one relies on (each
  // word's lowest bit holds the parity of the launch that wrote it), so nothing else may
  // write them: separate from `ptr`, which other calls reuse.
  static constexpr int kFusedSlots = 256, kFusedWords = 1024;
  static constexpr size_t kFusedBytes =
      ((size_t)kFusedSlots * 16 * 256 + (size_t)kFusedSlots * 16 * 2 + kFusedWords) * 4;
  void *fused = nullptr;
  int reserve(size_t need);
  int reserve_fused(hipStream_t s);  // allocates and zeroes `fused` once
  int reserve_host(size_t need);   // waits for the previous staged copy first
  int mark_host_used(hipStream_t s);
  ~Workspace();
};

}  // namespace pkv

struct pkv_rope {
  int n_rot;
  int64_t max_pos;
  float *cos, *sin;  // device [max_pos][n_rot / 2]
};

struct pkv_cache {
  int quant, batch, n_kv_heads, head_dim, padded;
  int64_t max_seq_len, seq_len;
  size_t bpr;
  uint8_t *k, *v;
  hipStream_t stream;
  hipEvent_t order_ev;  // orders a prefix restore (on another stream) with this stream
  pkv::Workspace ws;
  pkv::Workspace qws;  // prepared q of a decode step with q/k preparation
  pkv::RowStrides strides() const {
    return {(int64_t)n_kv_heads * (int64_t)bpr, (int64_t)batch * n_kv_heads * (int64_t)bpr,
            (int64_t)bpr};
  }
};

namespace pkv {

// ---- launchers (pkv_quant.hip) ----
// Quantize n new tokens of k and v ([batch, heads, n, head_dim] f32) into rows
// starting at token `t0` of the K and V buffers.
int launch_append(int quant, const float *k, const float *v, uint8_t *kc, uint8_t *vc,
                  int batch, int heads, int head_dim, int64_t n, int64_t t0, hipStream_t s);
// The same into the pages of a paged sequence: token t's rows sit in page
// page_tab[t >> page_lg] of the K and V planes (pages page_bytes apart), row t % 2^page_lg.
int launch_append_paged(int quant, const float *k, const float *v, uint8_t *kpool,
                        uint8_t *vpool, const int32_t *page_tab, int page_lg,
                        int64_t page_bytes, int heads, int head_dim, int64_t n, int64_t t0,
                        hipStream_t s);
// One token into each of n <= kAppendSeqs rows sets (k, v [n, heads, 1, head_dim]): row
// (b, h) at row_off[b] + h * bpr of each pool plane.
constexpr int kAppendSeqs = 32;
int launch_append_rows(int quant, const float *k, const float *v, uint8_t *kpool, uint8_t *vpool,
                       const int64_t *row_off, int n, int heads, int head_dim, hipStream_t s);
// Dequantize rows [0, S) to f32 [batch, heads, S, head_dim].
int launch_dequant(int quant, const uint8_t *kc, const uint8_t *vc, float *ko, float *vo,
                   int batch, int heads, int head_dim, int64_t S, hipStream_t s);

// ---- launcher (pkv_prep.hip) ----
// One launch: q rows [b, l, num_heads, d] -> q_norm + rope -> q_out; K rows
// [b, l, kv_heads, d] -> k_norm + rope -> encoded at cache token t0 + t; V rows encoded.
// Token t sits at position t0 + t of the rope tables.
struct PrepArgs {
  const float *q, *k, *v;  // q may be null (q_rows = 0)
  float *q_out;
  uint8_t *kc, *vc;
  const float *q_alpha, *k_alpha;   // [head_dim]
  const float *cos_tab, *sin_tab;   // [max_pos][n_rot / 2]
  float eps;
  int quant, batch, l, num_heads, kv_heads, head_dim, padded, n_rot;
  int64_t t0, bpr, q_rows, kv_rows;
};
int launch_prep_append(const PrepArgs &a, hipStream_t s);

// q/k preparation of a fused decode step (the Q4K MFMA decode kernel applies it itself).
struct DecodePrep {
  const float *q_alpha, *k_alpha;   // [256]
  const float *cos_tab, *sin_tab;   // [max_pos][n_rot / 2]
  float eps;
  int n_rot;
};

// ---- launchers (pkv_attn.hip) ----
struct AttnArgs {
  int quant;
  const float *q;  // [batch, l, num_heads, head_dim]
  const uint8_t *k, *v;
  RowStrides rs;
  float scale;
  int batch, num_heads, num_kv_heads, head_dim, l;
  int64_t seq_k, q_offset;
  int causal;
  float *out;  // [batch, l, num_heads, head_dim]
};
int launch_attend(const AttnArgs &a, Workspace &ws, hipStream_t s);

// Fused decode step: quantize one token (k, v [batch, heads, 1, head_dim]) into row
// t_new and attend over keys [0, t_new].
int launch_append_attend(const AttnArgs &a, const float *k_new, const float *v_new,
                         uint8_t *kc, uint8_t *vc, int64_t t_new, Workspace &ws,
                         hipStream_t s);

// Decode step from projection outputs: prepare q and the new k (see DecodePrep), quantize
// the new row into t_new and attend over keys [0, t_new], all inside the decode and combine
// kernels. PKV_ERR_UNSUPPORTED when the shape has no such kernel.
int launch_append_attend_prep_mfma(const AttnArgs &a, const float *k_new, const float *v_new,
                                   uint8_t *kc, uint8_t *vc, int64_t t_new,
                                   const DecodePrep &prep, Workspace &ws, hipStream_t s);

struct SeqDesc {
  uint8_t *k, *v;
  int64_t len;  // keys after the append
};
int launch_append_attend_batched(int quant, const SeqDesc *seqs_host, int n, const float *k,
                                 const float *v, const float *q, int num_heads,
                                 int num_kv_heads, int head_dim, float scale, float *out,
                                 Workspace &ws, hipStream_t s);

// ---- paged decode (pkv_attn_mfma.hip: Q4K, pkv_q8_decode.hip: Q8_0) ----
// Decode attention of nseq <= kMaxPagedSeqs paged sequences, one query each (q, out
// [nseq][16][256]), 16 query heads, 2 KV heads, head_dim 256, Q4K: sequence i attends to
// its len keys, held in the pages listed (device memory, in token order) at
// seqs[i].pages of the pool's K and V planes. Fused step (k_new non-null): the launch
// also quantizes each sequence's new token (k_new, v_new [nseq][2][256] f32) into row
// len of page pages[len >> page_lg] (allocated by the caller) and attends to it as well;
// a sequence may then hold no keys yet.
struct PagedSeqDesc {
  const int32_t *pages;
  int64_t len;
};
struct PagedPoolDesc {
  uint8_t *k, *v;  // planes: page p at p * page_bytes
  int64_t page_bytes;
  int page_lg;  // log2 tokens per page
};
constexpr int kMaxPagedSeqs = 32;
int launch_paged_decode_q4k(const PagedSeqDesc *seqs, int nseq, const PagedPoolDesc &pool,
                            const float *q, float *out, float scale, Workspace &ws,
                            hipStream_t s, const float *k_new = nullptr,
                            const float *v_new = nullptr);
// Q8_0: segs lists every page run, sequence by sequence (qi 0, 0, .., 1, ..), each at most
// page_tokens keys: rows of tokens [0, len) of the page (K and V planes, rows of head 1 at
// rs_h), for query / output row qi. More than 32 segments travel in a device table
// copied from `stage`, a pinned host buffer of at least nseg * kPagedSegBytes bytes that
// the caller keeps unchanged until the copy has run (it records an event after the call).
struct PagedSeg {
  uint8_t *k, *v;
  int64_t len;
  int qi;
};
constexpr int kPagedArgSegs = 32;  // segments carried in the kernel arguments
constexpr size_t kPagedSegBytes = 64;
int launch_paged_decode_q8(const PagedSeg *segs, int nseg, int nseq, int page_tokens,
                           const float *q, float *out, int64_t rs_t, int64_t rs_h, float scale,
                           void *stage, Workspace &ws, hipStream_t s);

// ---- launchers (pkv_util.hip) ----
int launch_fill_normal(float *dst, size_t n, uint64_t seed, uint64_t stream_id, float scale,
                       hipStream_t s);
int launch_scale_channels(float *x, size_t rows, int dim, const int *ch, int n_ch,
                          float factor, hipStream_t s);
int launch_copy_segments(void *const *dst, const void *const *src, const size_t *bytes, int n,
                         Workspace &ws, hipStream_t s);
// n words of dst set to zero by a kernel (capturable, unlike hipMemsetAsync).
int launch_zero_words(uint32_t *dst, size_t n, hipStream_t s);
int launch_oproj(const float *attn, const float *gate, const uint8_t *w, int w_type, float *out,
                 int batch, int in_dim, int out_dim, hipStream_t s);
// ---- launcher (pkv_oproj_mfma.hip): the batched form, Q4K/Q5K/Q6K ----
int launch_oproj_mfma(const float *attn, const float *gate, const uint8_t *w, int w_type,
                      float *out, int batch, int in_dim, int out_dim, Workspace &ws,
                      hipStream_t s);
int launch_deltanet_step(const float *q, const float *k, const float *v, const float *gate,
                         const float *beta, float *state, float *gate_offset, float *out,
                         int batch, int heads, int head_dim, float scale, float eps,
                         hipStream_t s);

}  // namespace pkv
