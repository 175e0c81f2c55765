/*
 * pkv_oracle — CPU restatement of paramecia-model's quantized KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY. This code is the checker for the HIP library in
 * paramecia_amd/; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it. The product path never calls it.
 *
 * What it restates (paths relative to the reference root):
 *   - KvCacheQuantization modes ............ paramecia-model/src/qwen3_next.rs:88-166
 *   - PreallocatedQuantizedKvCache ......... qwen3_next.rs:343-643 (new/append/get_kv/
 *                                            truncate/clear/resize_batch)
 *   - FullAttention cache offset rule ...... qwen3_next.rs:2430-2440
 *   - CPU SDPA (repeat_kv, scale, mask,
 *     clamp +-100, softmax, PV) ............ qwen3_next.rs:2580-2605, utils.rs:71-83,
 *                                            causal mask qwen3_next.rs:5022-5028
 *   - Q8_0 / Q4K codecs: the reference calls them through candle's
 *     QTensor::quantize / dequantize (qwen3_next.rs:486-487, 541-564). candle is an
 *     un-vendored git dependency (nicksenger/candle, branch paramecia, rev
 *     2278f29b93305e3d0d110149879175cea2898216, Cargo.lock:388-390) that is not
 *     present in this tree. The codecs below restate upstream candle's published
 *     k_quants.rs algorithm (BlockQ8_0::from_float/to_float, BlockQ4K::from_float
 *     with make_qkx1_quants(15, 5), BlockQ4K::to_float, get_scale_min_k4) and the
 *     `half` crate's f16/bf16 round-to-nearest-even conversion.
 *
 * Parity status (how each function is pinned; see tests/test_oracle_*.py):
 *   f16/bf16 conversion ....... pinned: exhaustive comparison against numpy's IEEE
 *                               float16 and a bit-level RNE bfloat16 definition.
 *   Q8_0 quantize/dequantize .. pinned: closed form per block, known-answer blocks
 *                               (zero block, +-amax -> +-127, exact .5 ties rounded
 *                               away from zero), idempotence of Q(DQ(.)).
 *   Q4K dequantize ............ pinned: GGML block layout closed form (hand-built
 *                               blocks with known scales/mins/nibbles).
 *   Q4K quantize .............. pinned against the published algorithm: hand-derived
 *                               known answers of make_qkx1_quants that take 3 to 5
 *                               passes, hit rounding ties and show the summation order
 *                               (tests/q4k_known_answers.py), a whole block built from
 *                               them, exact-grid blocks, format invariants and the
 *                               reconstruction error bound; each of seven planted
 *                               mistakes (pass count +-1, no early exit, ties to even,
 *                               pairwise sums, make_qkx2_quants, no min clamp; the
 *                               ORC_MUTANT builds) fails at least one known answer
 *                               (tests/test_oracle_mutants.py). The candle fork's own
 *                               bytes are absent; a divergence of the fork from upstream
 *                               candle would not show.
 *   cache layout/offsets ...... pinned: closed-form row addressing and the
 *                               overflow / offset-mismatch rules.
 *   attention ................. pinned: float64 restatement compared with an
 *                               independent numpy softmax(QK^T)V on small shapes.
 *   RNG ....................... pinned: Philox4x32-10 known-answer vectors from
 *                               Salmon et al. (SC'11) / Random123.
 *   rope tables ............... pinned: closed form inv_freq = theta^(-2i/n_rot)
 *                               against float64, position 0 -> (1, 0) exactly,
 *                               cos^2 + sin^2 = 1, and transformers' independent
 *                               Qwen3-Next rotary module (partial_rotary_factor).
 *   rms_norm .................. pinned: closed forms (constant row, one-hot row),
 *                               per-element alpha, float64 restatement, and
 *                               transformers' Qwen3NextRMSNorm (weight 1 + w).
 *   rope (half-split) ......... pinned: unit-vector rotations (sign and pairing
 *                               (i, i + n_rot/2)), position 0 = identity, pass-through
 *                               of dims >= n_rot, float64 complex rotation, and
 *                               transformers' apply_rotary_pos_emb.
 *   The last ulp of these three follows candle's CPU kernels (rms_norm,
 *   rotary_emb::rope) and the host libm's powf/sinf/cosf, restated; the candle fork
 *   is absent, so bit-level agreement with it is UNPINNED (tolerance-level pinned).
 *   Gated-DeltaNet step ....... pinned: transformers' torch_recurrent_gated_delta_rule
 *                               (FLA convention, state transposed), a float64
 *                               restatement, and closed forms (beta -> 0 is pure
 *                               decay; zero state gives sigmoid(b) v (k.q); a one-hot
 *                               key with beta = 1 writes v into that state column).
 *                               The fused CUDA kernel behind ops.rs:391-403 lives in
 *                               the absent candle fork, so its rounding is UNPINNED
 *                               (tolerance-level pinned).
 *   Q5K / Q6K dequantize ...... pinned against the published GGML block layouts (the
 *                               reference holds no Q5K/Q6K vectors): blocks packed element
 *                               by element decode bit-exactly to the closed form, single-bit
 *                               perturbations move exactly the element the layout names, a
 *                               Q5K block without high bits decodes as the Q4K block
 *                               (tests/test_oracle_kquants.py). The fork's decoders are
 *                               absent; a divergence of the fork from upstream would not show.
 *   gated o_proj (Q8_0/Q4K/Q5K/Q6K wo)
 *                               pinned: float64 numpy restatement of W_deq @ (x * sigmoid
 *                               (g)) with W_deq from the pinned dequantizers, and closed
 *                               forms (gate -> +inf passes x, -inf gives 0, 0 halves it).
 *                               The reference's QMatMul (candle fork, absent) may quantize x
 *                               before its dot products; that rounding is UNPINNED.
 */
#ifndef PKV_ORACLE_H
#define PKV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same numbering as include/pkv.h */
enum { ORC_F16 = 1, ORC_BF16 = 2, ORC_Q8_0 = 3, ORC_Q4K = 4 };
enum { ORC_OK = 0, ORC_ERR_OVERFLOW = 1, ORC_ERR_OFFSET = 2, ORC_ERR_ARG = 3 };
/* GGUF weight types of the output projection: GGML's ggml_type numbers */
enum { ORC_W_Q8_0 = 8, ORC_W_Q4K = 12, ORC_W_Q5K = 13, ORC_W_Q6K = 14 };

/* ---- scalar conversions (half crate semantics) ---- */
uint16_t orc_f32_to_f16(float x);
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float x);
float orc_bf16_to_f32(uint16_t h);
void orc_f32_to_f16_n(const float *x, uint16_t *out, size_t n);
void orc_f32_to_bf16_n(const float *x, uint16_t *out, size_t n);
void orc_f16_to_f32_n(const uint16_t *h, float *out, size_t n);

/* ---- codecs: n = elements, multiple of the block size ---- */
void orc_q8_0_quantize(const float *x, uint8_t *out, size_t n);
void orc_q8_0_dequantize(const uint8_t *in, float *y, size_t n);
void orc_make_qkx1_quants(const float *x, int n, int nmax, int ntry, float *scale,
                          float *neg_min);
void orc_get_scale_min_k4(int j, const uint8_t *scales, uint8_t *sc, uint8_t *m);
void orc_q4k_quantize(const float *x, uint8_t *out, size_t n);
void orc_q4k_dequantize(const uint8_t *in, float *y, size_t n);
void orc_q5k_dequantize(const uint8_t *in, float *y, size_t n); /* 176 B per 256 */
void orc_q6k_dequantize(const uint8_t *in, float *y, size_t n); /* 210 B per 256 */

/* ---- seeded synthetic data (identical on the GPU side) ---- */
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
float orc_normal(uint64_t seed, uint64_t stream, uint64_t index);
void orc_fill_normal(float *out, size_t n, uint64_t seed, uint64_t stream, float scale);

/* ---- preallocated quantized cache ---- */
typedef struct {
  int quant, batch, n_kv_heads, head_dim, padded_head_dim, block;
  int64_t max_seq_len, seq_len;
  size_t bytes_per_row;
  uint8_t *k, *v;
} orc_cache;

size_t orc_bytes_per_row(int quant, int head_dim);
int orc_cache_init(orc_cache *c, int quant, int batch, int n_kv_heads, int head_dim,
                   int64_t max_seq_len);
void orc_cache_free(orc_cache *c);
/* k, v: f32 [batch, n_kv_heads, n, head_dim] (the reference's append input). */
int orc_cache_append(orc_cache *c, const float *k, const float *v, int64_t n);
/* FullAttention rule: offset < len truncates, offset > len is an error. */
int orc_cache_append_at(orc_cache *c, const float *k, const float *v, int64_t n,
                        int64_t offset);
void orc_cache_truncate(orc_cache *c, int64_t new_len);
void orc_cache_clear(orc_cache *c);
int orc_cache_resize_batch(orc_cache *c, int batch);
/* get_kv: k_out, v_out f32 [batch, n_kv_heads, seq_len, head_dim]. */
void orc_cache_get_kv(const orc_cache *c, float *k_out, float *v_out);

/* ---- attention ----
 * q: f32 [batch, l, num_heads, head_dim]; out: f32 [batch, l, num_heads, head_dim].
 * Keys are the cache's first seq_len tokens. If causal, key j is visible to query i
 * iff j <= i + q_offset (the reference's causal_mask, qwen3_next.rs:5022-5028, which
 * its forward applies whenever l > 1; for l == 1 the mask hides nothing). Scores are
 * scaled, masked (-> -inf), clamped to [-100, 100] (so masked scores become -100
 * exactly as in the reference) and soft-maxed.
 * threads: 0 = all cores.
 */
int orc_attend_f32(const orc_cache *c, const float *q, int l, int num_heads, float scale,
                   int64_t q_offset, int causal, float *out, int threads);
int orc_attend_f64(const orc_cache *c, const float *q, int l, int num_heads, double scale,
                   int64_t q_offset, int causal, double *out);
/* Faithful cost structure of qwen3_next.rs:2470-2473 + 2580-2605 (dequantize the whole
 * cache, permute copy, repeat_kv copy, transposed-K copy, matmul, softmax, matmul). */
int orc_attend_faithful(const orc_cache *c, const float *q, int l, int num_heads,
                        float scale, int64_t q_offset, int causal, float *out, int threads);

/* ---- q/k preparation ahead of the cache (FullAttention::forward, qwen3_next.rs:2369-2399) ----
 * RotaryEmbedding::new (qwen3_next.rs:878-904): inv_freq[i] = 1 / (f32)(theta^(2i / n_rot))
 * with the power in f64, freqs[p][i] = (f32)p * inv_freq[i], cos/sin in f32 (libm cosf,
 * sinf). Tables are [max_pos][n_rot / 2]. n_rot must be even and positive. */
int orc_rope_tables(int n_rot, int64_t max_pos, double theta, float *cos_out, float *sin_out);
/* candle_nn::ops::rms_norm on the CPU: per row of d values, sum2 = sequential f32 sum of
 * x*x, m = sqrtf(sum2 / d + eps), y = x / m * alpha (qwen3_next.rs:2369, 2389). */
void orc_rms_norm(const float *x, const float *alpha, float eps, size_t rows, int d, float *y);
/* candle_nn::rotary_emb::rope (half-split pairs (i, i + n_rot/2)) on the first n_rot
 * values of each row of d values, in place; row r sits at position pos[r]
 * (RotaryEmbedding::apply, qwen3_next.rs:906-940). */
int orc_rope_rows(float *x, size_t rows, int d, int n_rot, const int64_t *pos,
                  const float *cos_tab, const float *sin_tab);
/* q: [batch, l, n_heads, d] -> q_norm then rope; k: [batch, l, n_kv_heads, d] -> k_norm
 * then rope; token t sits at position offset + t. Outputs keep the input layout. Either
 * of q / k may be NULL (with its output). */
int orc_qk_prep(const float *q, const float *k, int batch, int l, int n_heads, int n_kv_heads,
                int d, const float *q_alpha, const float *k_alpha, float eps, int n_rot,
                const float *cos_tab, const float *sin_tab, int64_t offset, float *q_out,
                float *k_out);

/* Gated-DeltaNet autoregressive step: candle::deltanet_ops::delta_net_autoregressive_step
 * (ops.rs:391-403) as the linear-attention layer calls it (qwen3_next.rs:3392-3470).
 * q, k: [batch, heads, d]; v: [batch, heads, d]; gate (log decay), beta (pre-sigmoid):
 * [batch, heads]; state: [batch, heads, d (v index i), d (k index j)], updated in place
 * (qwen3_next.rs:3634-3640 fixes the index roles: v_prime[i] = sum_j k[j] state[i][j]).
 * Per (b, h), in this order, f32:
 *   qn = q * scale / sqrtf(sum q*q + eps), kn = k / sqrtf(sum k*k + eps)
 *   S = S * exp(gate); u_i = sum_j S_ij kn_j; d_i = (v_i - u_i) * sigmoid(beta)
 *   S_ij = S_ij + kn_j d_i; out_i = sum_j S_ij qn_j
 * and gate_offset[b, h] += gate (the gate_cumsum_offset update, qwen3_next.rs:3444-3451;
 * gate_offset may be NULL). Sums run in index order. */
void orc_deltanet_step(const float *q, const float *k, const float *v, const float *gate,
                       const float *beta, float *state, float *gate_offset, float *out,
                       int batch, int heads, int d, float scale, float eps);

/* Gated output projection (qwen3_next.rs:2657-2680): y = x * sigmoid(g) (f32:
 * 1 / (1 + expf(-g)), gate may be NULL), then out[b][o] = sum_i Wdq[o][i] y[i] with Wdq the
 * rows of w (out_dim rows of in_dim elements in GGUF type w_type, ORC_W_*) dequantized by
 * the matching orc_*_dequantize, summed in index order in f32. ORC_ERR_ARG for an unknown
 * type or an in_dim that is not a whole number of blocks. */
size_t orc_weight_row_bytes(int w_type, int in_dim);
int orc_gated_oproj(const float *attn, const float *gate, const uint8_t *w, int w_type,
                    float *out, int batch, int in_dim, int out_dim);
void orc_gated_oproj_q4k(const float *attn, const float *gate, const uint8_t *w, float *out,
                         int batch, int in_dim, int out_dim);

#ifdef __cplusplus
}
#endif
#endif
