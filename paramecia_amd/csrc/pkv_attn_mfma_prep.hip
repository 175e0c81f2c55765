// Q4K MFMA decode step from projection outputs: the decode kernel of pkv_q4k_decode.hpp
// instantiated with q_norm / k_norm / rope inside (kPrep = true). A translation unit of
// its own, so that this instantiation and the plain one are optimised separately.
#include "pkv_q4k_decode.hpp"

namespace pkv {

int launch_append_attend_prep_mfma(const AttnArgs &a, const float *k_new, const float *v_new,
                                   uint8_t *kc, uint8_t *vc, int64_t t_new,
                                   const DecodePrep &prep, Workspace &ws, hipStream_t s) {
  if (a.quant != PKV_QUANT_Q4K || a.head_dim != 256 || a.num_heads != 16 ||
      a.num_kv_heads != 2 || a.l != 1)
    return PKV_ERR_UNSUPPORTED;
  // the rope pairs (j, j + 32) of n_rot = 64 (Qwen3-Next) sit in one lane of build_q
  if (prep.n_rot != 64) return PKV_ERR_UNSUPPORTED;
  if (kc != a.k || vc != a.v || t_new != a.seq_k - 1 || a.q_offset != t_new)
    return PKV_ERR_UNSUPPORTED;
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
    const int rc = launch_decode_segments<true>(in, nb, a.q + qo, k_new + ko, v_new + ko, a.out + qo,
                                          a.rs.t, a.rs.h, a.scale, ws, s, &prep);
    if (rc) return rc;
  }
  return PKV_OK;
}

}  // namespace pkv
