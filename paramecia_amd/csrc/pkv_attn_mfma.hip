// Q4K MFMA decode launchers (decode kernel without q/k preparation); the kernel, its
// helpers and the launch plan are in pkv_q4k_decode.hpp.
#include "pkv_q4k_decode.hpp"

namespace pkv {

int launch_attend_mfma(const AttnArgs &a, const float *k_new, const float *v_new, uint8_t *kc,
                       uint8_t *vc, int64_t t_new, Workspace &ws, hipStream_t s) {
  if (a.quant != PKV_QUANT_Q4K || a.head_dim != 256 || a.num_heads != 16 ||
      a.num_kv_heads != 2 || a.l != 1)
    return PKV_ERR_UNSUPPORTED;
  // decode only: the single query sees every key
  if (a.causal && a.q_offset + 1 < a.seq_k) return PKV_ERR_UNSUPPORTED;
  const bool fused = k_new != nullptr;
  // the fused step writes the new row into the cache being read, at its last row
  if (fused && (kc != a.k || vc != a.v || t_new != a.seq_k - 1)) return PKV_ERR_UNSUPPORTED;
  if (!decode_rows_fit(a.seq_k, a.rs.t)) return PKV_ERR_UNSUPPORTED;
  for (int b0 = 0; b0 < a.batch; b0 += kMaxSegs) {
    const int nb = a.batch - b0 < kMaxSegs ? a.batch - b0 : kMaxSegs;
    DecodeSegIn in[kMaxSegs];
    for (int i = 0; i < nb; ++i) {
      in[i].k = const_cast<uint8_t *>(a.k) + (int64_t)(b0 + i) * a.rs.b;
      in[i].v = const_cast<uint8_t *>(a.v) + (int64_t)(b0 + i) * a.rs.b;
      in[i].seq_k = a.seq_k;
    }
    const int64_t qo = (int64_t)b0 * 16 * 256, ko = (int64_t)b0 * 2 * 256;
    const int rc = launch_decode_segments<false>(in, nb, a.q + qo, fused ? k_new + ko : nullptr,
                                          fused ? v_new + ko : nullptr, a.out + qo, a.rs.t,
                                          a.rs.h, a.scale, ws, s);
    if (rc) return rc;
  }
  return PKV_OK;
}

int launch_append_attend_batched_mfma(int quant, const SeqDesc *seqs, int n, const float *k,
                                      const float *v, const float *q, int num_heads,
                                      int num_kv_heads, int head_dim, float scale, float *out,
                                      Workspace &ws, hipStream_t s) {
  if (quant != PKV_QUANT_Q4K || head_dim != 256 || num_heads != 16 || num_kv_heads != 2)
    return PKV_ERR_UNSUPPORTED;
  const int64_t rs_t = 2 * 144, rs_h = 144;
  for (int i = 0; i < n; ++i)
    if (seqs[i].len < 1 || !decode_rows_fit(seqs[i].len, rs_t)) return PKV_ERR_UNSUPPORTED;
  for (int b0 = 0; b0 < n; b0 += kMaxSegs) {
    const int nb = n - b0 < kMaxSegs ? n - b0 : kMaxSegs;
    DecodeSegIn in[kMaxSegs];
    for (int i = 0; i < nb; ++i) {
      in[i].k = seqs[b0 + i].k;
      in[i].v = seqs[b0 + i].v;
      in[i].seq_k = seqs[b0 + i].len;
    }
    const int64_t qo = (int64_t)b0 * 16 * 256, ko = (int64_t)b0 * 2 * 256;
    const int rc = launch_decode_segments<false>(in, nb, q + qo, k + ko, v + ko, out + qo, rs_t, rs_h,
                                          scale, ws, s);
    if (rc) return rc;
  }
  return PKV_OK;
}

}  // namespace pkv
