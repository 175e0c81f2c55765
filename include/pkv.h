/*
 * pkv.h — C ABI of the MI355X-native quantized KV-cache library (libpkv.so).
 *
 * Drop-in boundary for paramecia-model's full-attention KV-cache path. Each entry
 * point names the reference item it replaces (paths relative to the reference root,
 * mostly paramecia-model/src/qwen3_next.rs, "qn" below).
 *
 * Conventions
 *   - All tensor arguments are DEVICE pointers (hipMalloc'd or torch CUDA tensors),
 *     plain C types only. Host-side bookkeeping (lengths, tokens) is plain values.
 *   - Every call returns an int status (pkv_status); on failure
 *     pkv_last_error() returns a thread-local message. Nothing is partially
 *     written on a returned error (the reference's bail! semantics).
 *   - A cache handle owns its K/V buffers and a stream (hipStream_t passed as
 *     void*; NULL = the default stream). Work is enqueued on that stream and
 *     returns without synchronising. A handle is not re-entrant (the reference
 *     holds the cache behind &mut self); different handles are independent.
 *   - Layout in HBM is the reference's seq-major row layout (qn:465-504): row
 *     r = (t*batch + b)*n_kv_heads + h, row r at byte r*bytes_per_row in the K and
 *     in the V buffer. One row = one head of one token = padded_head_dim elements
 *     in GGML blocks (Q4K: 144 B per 256, Q8_0: 34 B per 32) or f16/bf16.
 */
#ifndef PKV_H
#define PKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct pkv_cache pkv_cache;   /* PreallocatedQuantizedKvCache (qn:343-380) */
typedef struct pkv_prefix pkv_prefix; /* PrefixCache (qn:856-864) */
typedef void *pkv_stream;             /* hipStream_t */

/* KvCacheQuantization (qn:88-106). NONE is the deprecated alias of F16. */
enum {
  PKV_QUANT_NONE = 0,
  PKV_QUANT_F16 = 1,
  PKV_QUANT_BF16 = 2,
  PKV_QUANT_Q8_0 = 3,
  PKV_QUANT_Q4K = 4
};

enum {
  PKV_OK = 0,
  PKV_ERR_OVERFLOW = 1,   /* "Quantized KV cache overflow" (qn:435-441) */
  PKV_ERR_OFFSET = 2,     /* "KV cache offset mismatch" (qn:2430-2440) */
  PKV_ERR_ARG = 3,        /* bad argument / shape */
  PKV_ERR_HIP = 4,        /* HIP runtime error */
  PKV_ERR_EMPTY = 5,      /* "Cannot get storage from empty cache" (qn:583-585) */
  PKV_ERR_LAYERS = 6,     /* "Prefix cache layer count mismatch" (qn:5727-5733) */
  PKV_ERR_LAYOUT = 7,     /* snapshot does not fit the cache (quant/heads/dims) */
  PKV_ERR_UNSUPPORTED = 8 /* combination with no kernel (e.g. head_dim > 512), or a call that
                             allocates, made on a capturing stream */
};

/* Entry kinds of a prefix cache layer (PrefixCacheEntry, qn:834-854). */
enum { PKV_ENTRY_EMPTY = 0, PKV_ENTRY_FULL = 1, PKV_ENTRY_LINEAR = 2 };

/* Restore modes for pkv_prefix_restore. BYTES copies the packed blocks (bit-exact);
 * REQUANTIZE reproduces the reference's clear()+append(dequantized) (qn:2843-2847). */
enum { PKV_RESTORE_BYTES = 0, PKV_RESTORE_REQUANTIZE = 1 };

const char *pkv_last_error(void);
const char *pkv_version(void);
/* Waits for the current device, then reports and clears the errors its kernels flagged
 * instead of hanging: PKV_ERR_HIP if a fused decode step's bounded barrier gave up (the
 * step's appended row and output are then invalid), PKV_OK otherwise. No reference
 * counterpart (the reference's CPU path cannot hang a barrier). */
int pkv_device_status(void);

/* ---- KvCacheQuantization helpers (qn:107-166) ---- */
/* from_str: f16|fp16, bf16|bfloat16, q8|q8_0, q4|q4k|q4_k, none (case-insensitive). */
int pkv_quant_parse(const char *s, int *quant_out);
int pkv_quant_default(void);                  /* impl Default -> Q4K (qn:107-111) */
int pkv_quant_block_size(int quant);          /* block_size() (qn:123-130) */
int pkv_quant_is_ggml(int quant);             /* to_ggml_dtype().is_some() (qn:114-121) */
size_t pkv_bytes_per_row(int quant, int head_dim); /* qn:393-402 */

/* ---- cache lifecycle (qn:384-423, 620-642) ---- */
int pkv_create(int quant, int batch, int n_kv_heads, int head_dim, int64_t max_seq_len,
               pkv_stream stream, pkv_cache **out);
int pkv_destroy(pkv_cache *h);
int pkv_set_stream(pkv_cache *h, pkv_stream stream);
int64_t pkv_len(const pkv_cache *h);            /* seq_len */
int64_t pkv_capacity(const pkv_cache *h);       /* max_seq_len */
int pkv_geometry(const pkv_cache *h, int *quant, int *batch, int *n_kv_heads, int *head_dim,
                 size_t *bytes_per_row);
int pkv_truncate(pkv_cache *h, int64_t new_len); /* truncate(): min(new_len, len) */
/* LayerWeights::restore_cache (qn:4326-4337) assigns seq_len directly: len may exceed the
 * current length (the rows past it are whatever the buffers hold), not the capacity
 * (PKV_ERR_OVERFLOW). */
int pkv_set_len(pkv_cache *h, int64_t len);
int pkv_clear(pkv_cache *h);                     /* clear() */
int pkv_resize_batch(pkv_cache *h, int batch);   /* resize_batch(): realloc + reset if changed */

/* ---- append (append_quantized qn:431-509 + FullAttention offset rule qn:2430-2440) ----
 * k, v: device f32 [batch, n_kv_heads, n, head_dim]. offset < len truncates first,
 * offset > len -> PKV_ERR_OFFSET, len+n > capacity -> PKV_ERR_OVERFLOW. Pass
 * offset = -1 to append at the current length. */
int pkv_append(pkv_cache *h, const float *k, const float *v, int64_t n, int64_t offset);

/* ---- attention over the cache (CPU SDPA qn:2580-2605, flash_attn_q8 role qn:2531-2561) ----
 * q, out: device f32 [batch, l, num_heads, head_dim]. Query head g reads KV head
 * g / (num_heads / n_kv_heads) (repeat_kv, utils.rs:71-83). Key j is visible to query
 * i iff !causal or j <= i + q_offset; scores are scaled, clamped to [-100, 100] and
 * soft-maxed. For the model path q_offset = len - l and causal = 1 (qn:2538-2542). */
int pkv_attend(pkv_cache *h, const float *q, int l, int num_heads, float scale,
               int64_t q_offset, int causal, float *out);

/* One decode step of one full-attention layer: append one token (offset rule as
 * pkv_append) then attend over all len+1 keys, in one call.
 * k, v: [batch, n_kv_heads, 1, head_dim]; q, out: [batch, 1, num_heads, head_dim]. */
int pkv_append_attend(pkv_cache *h, const float *k, const float *v, const float *q,
                      int num_heads, float scale, int64_t offset, float *out);

/* get_kv (qn:520-575): dequantize rows [0, len) into device f32
 * [batch, n_kv_heads, len, head_dim] (padding trimmed). */
int pkv_get_kv(pkv_cache *h, float *k_out, float *v_out);

/* get_kv_storage (qn:582-617): device pointers to the packed K/V bytes, the valid
 * byte count, and the byte strides of the [batch, seq, head, d] view
 * (stride_b, stride_seq, stride_h, stride_d). Empty cache -> PKV_ERR_EMPTY. */
int pkv_kv_storage(const pkv_cache *h, const void **k_bytes, const void **v_bytes,
                   size_t *valid_bytes, int64_t strides[4]);

/* flash_attn_q8 (paramecia-model/src/ops.rs:756-792), stateless, any of the four
 * storage formats: K/V are packed rows addressed by the byte strides
 * (stride_b, stride_seq, stride_h) as returned by pkv_kv_storage. */
int pkv_flash_attn(int quant, const float *q, const void *k_bytes, const void *v_bytes,
                   const int64_t kv_strides[3], float scale, int batch, int num_heads,
                   int num_kv_heads, int head_dim, int seq_q, int64_t seq_k,
                   int64_t q_offset, int causal, float *out, pkv_stream stream);

/* pkv_flash_attn for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). It has no counterpart
 * in the reference. Same arguments, kernels and results as pkv_flash_attn, but the
 * split-K partials go to a library-owned static device array of
 * PKV_NOALLOC_SCRATCH_BYTES on the current device (each GPU holds its own copy until the
 * process ends) instead of an allocated workspace: the call allocates nothing, and a
 * call whose work plan needs more scratch returns PKV_ERR_ARG before it enqueues
 * anything. `stream` must belong to the current device. Every call on one GPU shares that
 * GPU's array: calls that overlap in time on one GPU (other streams, other threads) race. */
#define PKV_NOALLOC_SCRATCH_BYTES (16u << 20)
int pkv_flash_attn_noalloc(int quant, const float *q, const void *k_bytes, const void *v_bytes,
                           const int64_t kv_strides[3], float scale, int batch, int num_heads,
                           int num_kv_heads, int head_dim, int seq_q, int64_t seq_k,
                           int64_t q_offset, int causal, float *out, pkv_stream stream);

/* Batched decode over independent sequences (serving loop): caches[i] is a batch-1
 * cache; appends one token to each (k, v: [n, n_kv_heads, head_dim]) then attends
 * (q, out: [n, num_heads, head_dim]). All caches share geometry. For the Qwen3-Next
 * shape (Q4K or Q8_0) up to 32 sequences share one decode + combine launch pair. */
int pkv_append_attend_batched(pkv_cache *const *caches, int n, const float *k,
                              const float *v, const float *q, int num_heads, float scale,
                              float *out, pkv_stream stream);

/* ---- q/k preparation fused into the append (FullAttention::forward qn:2369-2399) ----
 * RotaryEmbedding (qn:866-940): cos/sin tables [max_pos][n_rot/2] f32, built on the host
 * as RotaryEmbedding::new does (inv_freq = 1/theta^(2i/n_rot), f32 cos/sin of t*inv_freq)
 * and kept on the device; one table serves every layer (the reference shares it). */
typedef struct pkv_rope pkv_rope;
/* The tables alone, into host memory (no device work). */
int pkv_rope_tables_host(int n_rot, int64_t max_pos, double theta, float *cos_out,
                         float *sin_out);
int pkv_rope_create(int n_rot, int64_t max_pos, double theta, pkv_rope **out);
int pkv_rope_destroy(pkv_rope *r);
int pkv_rope_geometry(const pkv_rope *r, int *n_rot, int64_t *max_pos, const float **cos_tab,
                      const float **sin_tab);

/* One layer's q/k preparation: the RmsNorm alphas of attn_q_norm / attn_k_norm (device f32
 * [head_dim], qn:2297-2306), rms_norm_eps, and the shared rope. */
typedef struct {
  const float *q_alpha;
  const float *k_alpha;
  float eps;
  const pkv_rope *rope;
} pkv_qk_prep;

/* q_norm, k_norm, the [b,l,h,d] -> [b,h,l,d] transposes, rope (qn:2369-2399) and
 * append_quantized (qn:2442) in one launch. Inputs are the projection outputs as the
 * reference reshapes them: q [batch, n, num_heads, head_dim] (may be NULL, with q_out),
 * k, v [batch, n, n_kv_heads, head_dim]. q_out (same layout as q) receives the normalised,
 * rotated q; K rows are normalised and rotated, V rows taken as given, both encoded at
 * the cache's position. Token t sits at rope position offset + t (len + t for
 * offset = -1); positions past the rope table -> PKV_ERR_ARG before anything changes.
 * Offset, overflow and error rules otherwise as pkv_append. */
int pkv_append_prep(pkv_cache *h, const pkv_qk_prep *prep, const float *q, int num_heads,
                    float *q_out, const float *k, const float *v, int64_t n, int64_t offset);

/* A decode step from the projection outputs: pkv_append_prep of one token (its q into
 * the handle's scratch), then attention of the prepared q over all len+1 keys.
 * q, out: [batch, 1, num_heads, head_dim]; k, v: [batch, 1, n_kv_heads, head_dim]. */
int pkv_append_attend_prep(pkv_cache *h, const pkv_qk_prep *prep, const float *q,
                           const float *k, const float *v, int num_heads, float scale,
                           int64_t offset, float *out);

/* ---- PrefixCache (qn:834-864, 2780-2884, 4066-4132, 5702-5750) ---- */
int pkv_prefix_create(const uint32_t *prefix_tokens, size_t n_tokens, int n_layers,
                      pkv_prefix **out);
int pkv_prefix_free(pkv_prefix *p);
int pkv_prefix_tokens(const pkv_prefix *p, const uint32_t **tokens, size_t *n_tokens);
int pkv_prefix_num_layers(const pkv_prefix *p);
int pkv_prefix_entry_kind(const pkv_prefix *p, int layer);
/* save_kv_state (qn:2780-2815): snapshot rows [0, len) byte for byte (Empty if len 0). */
int pkv_prefix_save_full(pkv_prefix *p, int layer, const pkv_cache *h);
/* save_state_for_prefix (qn:4066-4104): deep copy of the Gated-DeltaNet state.
 * ssm [b, heads, dk, dv], conv [b, conv_dim, k-1], gate_offset [b, heads] f32;
 * gate_offset == NULL stores zeros (qn:4077-4093). */
int pkv_prefix_save_linear(pkv_prefix *p, int layer, const float *ssm, size_t n_ssm,
                           const float *conv, size_t n_conv, const float *gate_offset,
                           size_t n_gate, pkv_stream stream);
/* Saved element counts of a LINEAR entry (to size restore targets). */
int pkv_prefix_linear_sizes(const pkv_prefix *p, int layer, size_t *n_ssm, size_t *n_conv,
                            size_t *n_gate);
/* Saved length of a FULL entry. */
int64_t pkv_prefix_full_len(const pkv_prefix *p, int layer);

/* Restore targets for one layer: exactly one of `cache` (full attention) or the three
 * state pointers (linear attention) is set. The state pointers come with their capacities
 * in f32 elements; a LINEAR entry whose saved counts exceed them -> PKV_ERR_LAYOUT before
 * anything is written. `*state_valid` is written 1 if the state was restored, 0 if it was
 * cleared (Empty or wrong entry kind, qn:4121-4130). */
typedef struct {
  pkv_cache *cache;
  float *ssm;
  float *conv;
  float *gate_offset;
  int *state_valid;
  size_t ssm_cap, conv_cap, gate_cap;
} pkv_layer_target;

/* restore_prefix_cache (qn:5726-5740): layer count must match (PKV_ERR_LAYERS);
 * every layer is validated before anything is written; all copies go out as ONE
 * batched gather/copy launch on `stream`. FULL entries restore into the cache
 * (len = saved len), Empty/wrong-kind clear it (qn:2874-2882). Writes the prefix
 * token count to *n_tokens_out. mode: PKV_RESTORE_BYTES or PKV_RESTORE_REQUANTIZE.
 * Ordering: the launch waits for the snapshot's own copies (issued on the stream of
 * the save call) and for work already queued on each target cache's stream, and each
 * target cache's stream waits for the launch before its next work. */
int pkv_prefix_restore(const pkv_prefix *p, const pkv_layer_target *targets, int n_layers,
                       int mode, size_t *n_tokens_out, pkv_stream stream);

/* ---- Gated-DeltaNet recurrent state (the linear-attention layers) ---- */
/* delta_net_autoregressive_step (ops.rs:391-403) as delta_net_autoregressive calls it
 * (qwen3_next.rs:3392-3470): one token, in place. q, k, v: [batch, heads, head_dim]
 * (q, k already repeated to the value heads); gate (log decay) and beta (pre-sigmoid):
 * [batch, heads]; state: [batch, heads, head_dim (value i), head_dim (key j)], the
 * ssm_state of RecurrentState (qn:683-700); gate_offset: [batch, heads] or NULL, the
 * gate_cumsum_offset += gate update (qn:3444-3451); out: [batch, heads, head_dim].
 * qn = q*scale/sqrt(|q|^2+eps), kn = k/sqrt(|k|^2+eps); S *= exp(gate);
 * S_i += (v_i - S_i.kn) sigmoid(beta) kn; out_i = S_i.qn. head_dim 64, 128 or 256
 * (else PKV_ERR_UNSUPPORTED); q, k, state 16-byte aligned. A zero state stands for the
 * reference's missing state (qn:3424-3431). */
int pkv_deltanet_step(const float *q, const float *k, const float *v, const float *gate,
                      const float *beta, float *state, float *gate_offset, float *out,
                      int batch, int heads, int head_dim, float scale, float eps,
                      pkv_stream stream);

/* ---- the step after the attention ---- */
/* Gated output projection (qn:2657-2680): out[b][o] = sum_i W[o][i] * attn[b][i] *
 * sigmoid(gate[b][i]), W the layer's GGUF Q4K attn_output weight (self.wo, a QMatMul,
 * models/with_tracing.rs:253-300 without custom scales or LoRA): out_dim rows of
 * in_dim / 256 superblocks of 144 B. attn, gate: [batch, in_dim] f32 (gate may be NULL:
 * no gating); out: [batch, out_dim]. in_dim 4096 or 8192 (else PKV_ERR_UNSUPPORTED);
 * attn, gate and W 16-byte aligned. */
int pkv_gated_oproj_q4k(const float *attn, const float *gate, const void *w_q4k, float *out,
                        int batch, int in_dim, int out_dim, pkv_stream stream);

/* GGUF weight types of the output projection: GGML's ggml_type numbers, as a GGUF file
 * stores them per tensor (the reference's GgmlDType of self.wo, qn:1412-1413). */
enum { PKV_WTYPE_Q8_0 = 8, PKV_WTYPE_Q4K = 12, PKV_WTYPE_Q5K = 13, PKV_WTYPE_Q6K = 14 };

/* The same gated projection for any of the k-quant types a GGUF Qwen3-Next checkpoint
 * stores attn_output in (Q4K, Q5K, Q6K; Q8_0 checkpoints): W is out_dim rows of in_dim
 * elements of type w_type (Q4K 144 B, Q5K 176 B, Q6K 210 B per 256 inputs; Q8_0 34 B per
 * 32), the GGUF tensor bytes as stored. Same shapes and alignment as
 * pkv_gated_oproj_q4k; another w_type -> PKV_ERR_UNSUPPORTED. w_type Q4K is
 * pkv_gated_oproj_q4k. */
int pkv_gated_oproj(const float *attn, const float *gate, const void *w, int w_type, float *out,
                    int batch, int in_dim, int out_dim, pkv_stream stream);

/* ---- PrefixCache host spill (the survey's next row after the path: the reference keeps
 * prefixes in device memory only, qn:856-864; LocalBackend, paramecia-llm, is the caller
 * that would evict them). A blob is a self-describing host byte image of a prefix:
 * header, tokens, one descriptor per layer, then the packed K/V rows and DeltaNet states
 * exactly as saved. serialize first waits for the device (the snapshot copies ran on the
 * caches' streams), then copies device -> host on `stream` and waits for it;
 * deserialize checks every length and bound of the blob before it allocates, then
 * copies host -> device and waits. A bad or truncated blob -> PKV_ERR_ARG. */
size_t pkv_prefix_serialized_size(const pkv_prefix *p);
int pkv_prefix_serialize(const pkv_prefix *p, void *host_dst, size_t capacity, pkv_stream stream);
int pkv_prefix_deserialize(const void *host_src, size_t n, pkv_prefix **out, pkv_stream stream);

/* ---- Paged KV caches for multi-sequence serving (the survey's next row after the path:
 * the reference preallocates one PreallocatedQuantizedKvCache per layer and sequence at
 * max_seq_len, qn:343-380, and its serving caller LocalBackend keeps one sequence with a
 * deep-copied prefix, paramecia-llm/src/backend/local.rs:743-800). A pool holds n_pages
 * pages of page_tokens tokens (a power of two in [32, 2^20]) for one layer; a page is the
 * K and V rows of page_tokens tokens x n_kv_heads in the pool's encoding (PKV_QUANT_*),
 * laid out as a batch-1 cache of that capacity. A sequence is a list of pages. Work runs
 * on the pool's stream, in order. Not thread-safe: one host thread per pool. */
typedef struct pkv_pool pkv_pool;
typedef struct pkv_seq pkv_seq;
int pkv_pool_create(int quant, int n_kv_heads, int head_dim, int page_tokens, int n_pages,
                    pkv_stream stream, pkv_pool **out);
/* PKV_ERR_ARG while the pool still has sequences. */
int pkv_pool_destroy(pkv_pool *p);
int pkv_pool_free_pages(const pkv_pool *p);
/* The stream later work on the pool's sequences is queued on (the caller orders it after
 * work on the previous stream). */
int pkv_pool_set_stream(pkv_pool *p, pkv_stream stream);
int pkv_seq_create(pkv_pool *p, pkv_seq **out);
/* Waits for the pool's stream, then returns the sequence's pages. */
int pkv_seq_destroy(pkv_seq *s);
int64_t pkv_seq_len(const pkv_seq *s);
int pkv_seq_pages(const pkv_seq *s);
/* A new sequence sharing every page of s (no copy; a shared, partly filled last page is
 * copied when either sequence first appends into it). A prefix cache entry kept as a
 * sequence is restored by a fork. */
int pkv_seq_fork(const pkv_seq *s, pkv_seq **out);
/* Keep tokens [0, new_len) (new_len >= len: no change); whole pages past it return to the
 * pool. */
int pkv_seq_truncate(pkv_seq *s, int64_t new_len);
/* append_quantized (qn:431-509) into the sequence's pages: k, v [1, n_kv_heads, n,
 * head_dim] f32; offset as pkv_append (-1 appends at the end, a smaller offset rewinds,
 * a larger one -> PKV_ERR_OFFSET). PKV_ERR_OVERFLOW, with nothing written, when the
 * pool lacks pages. */
int pkv_seq_append(pkv_seq *s, const float *k, const float *v, int64_t n, int64_t offset);
/* One token appended to each of n sequences of one pool in one launch (the decode step of
 * a serving batch): k, v [n, n_kv_heads, 1, head_dim] f32. All or nothing: PKV_ERR_OVERFLOW,
 * with nothing written, when the pool lacks pages for any of them. */
int pkv_seq_append_batched(pkv_seq *const *seqs, int n, const float *k, const float *v);
/* Attention over the sequence's keys, as pkv_attend: q [1, l, num_heads, head_dim],
 * out the same shape. */
int pkv_seq_attend(pkv_seq *s, const float *q, int l, int num_heads, float scale,
                   int64_t q_offset, int causal, float *out);
/* One decode query per sequence (varlen), all sequences in one pool: q, out
 * [n, num_heads, head_dim]; each sees all its keys. Q4K / Q8_0 pools of the model's shape
 * (16 query heads, 2 KV heads, head_dim 256) run one decode launch per 32 sequences over
 * all their pages; other pools attend sequence by sequence. */
int pkv_seq_decode_batched(pkv_seq *const *seqs, int n, const float *q, int num_heads,
                           float scale, float *out);
/* The fused decode step of a serving batch (the paged form of pkv_append_attend_batched):
 * one token appended to each of n sequences of one pool (k, v [n, n_kv_heads, 1,
 * head_dim] f32), then one decode query per sequence over all its keys, the new one
 * included (q, out [n, num_heads, head_dim]). Q4K pools of the model's shape run one
 * decode launch per 32 sequences that also quantizes the new rows (kernel arguments and
 * the sequences' device page lists only: a step in which no sequence's page list changes
 * can be captured in a HIP graph; one that must copy a changed list returns
 * PKV_ERR_UNSUPPORTED under capture); other pools run pkv_seq_append_batched then
 * pkv_seq_decode_batched. All or nothing: PKV_ERR_OVERFLOW, with nothing written, when
 * the pool lacks pages for any of them. */
int pkv_seq_append_decode_batched(pkv_seq *const *seqs, int n, const float *k, const float *v,
                                  const float *q, int num_heads, float scale, float *out);
/* get_kv (qn:520-575): dequantized [1, n_kv_heads, len, head_dim] f32. */
int pkv_seq_get_kv(const pkv_seq *s, float *k_out, float *v_out);

/* ---- utilities ---- */
/* Seeded synthetic data: dst[i] = normal(seed, stream_id, i) * scale, bit-identical
 * to the CPU oracle's generator (Philox4x32-10, Irwin-Hall of eight 22-bit draws). */
int pkv_fill_normal(float *dst, size_t n, uint64_t seed, uint64_t stream_id, float scale,
                    pkv_stream stream);
/* Multiply channels ch[0..n_ch) of the last dimension (size dim) by factor. */
int pkv_scale_channels(float *x, size_t rows, int dim, const int *channels_host, int n_ch,
                       float factor, pkv_stream stream);
/* Device-to-device gather/copy of n segments in one launch (used by prefix restore). */
int pkv_copy_segments(void *const *dst, const void *const *src, const size_t *bytes, int n,
                      pkv_stream stream);

#ifdef __cplusplus
}
#endif
#endif /* PKV_H */
