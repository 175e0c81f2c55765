// Q4K MFMA decode launchers (decode kernel without q/k preparation); the kernel, its
// helpers and the launch plan are in pkv_q4k_decode.hpp.
#include <cstring>
#include <vector>

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

// Paged decode over device page lists: sequence i's segments are its pages (one virtual
// block for a sequence without keys), laid on one virtual block line with a gap before
// every segment after the first (the estimated cost of one more pass), split stream-K
// over the workgroups; the kernel derives its pieces and their pages from the
// per-sequence arguments, so nothing is copied to the device per call. Partial slots:
// workgroup w's pieces take w + (segment index), the slot after its last piece gets an
// empty partial when its range ends outside a segment, so a sequence's slots run from
// its first segment's first piece to its last segment's last piece with none unwritten.
int launch_paged_decode_q4k(const PagedSeqDesc *seqs, int nseq, const PagedPoolDesc &pool,
                            const float *q, float *out, float scale, Workspace &ws,
                            hipStream_t s, const float *k_new, const float *v_new) {
  const int64_t ptok = (int64_t)1 << pool.page_lg;
  const int64_t rs_t = 2 * 144, rs_h = 144;
  if (nseq < 1 || nseq > kMaxPagedSeqs || pool.page_lg < 5 || pool.page_lg > 20)
    return set_error(PKV_ERR_ARG, "paged decode: bad plan");
  if (!decode_rows_fit(ptok, rs_t)) return PKV_ERR_UNSUPPORTED;
  const bool fused = k_new != nullptr;
  if (fused && v_new == nullptr) return set_error(PKV_ERR_ARG, "paged decode: no new V rows");
  const int pblk = (int)(ptok / kBlk), pstride = pblk + kPieceGap;
  DecodeArgsT<0> d;
  CombineArgs c;
  int V = 0, K = 0;
  int vend[kMaxPagedSeqs];
  for (int i = 0; i < nseq; ++i) {
    const int64_t len = seqs[i].len;
    if (len < 0 || (len == 0 && !fused) || seqs[i].pages == nullptr)
      return set_error(PKV_ERR_ARG, "paged decode: a sequence without keys");
    const int64_t npg64 = len > 0 ? (len + ptok - 1) / ptok : 1;
    if (npg64 > (1 << 20) || (int64_t)V + npg64 * pstride + kPieceGap >= (1 << 30))
      return set_error(PKV_ERR_ARG, "paged decode: too many pages");
    const int npg = (int)npg64;
    if (i > 0) V += kPieceGap;
    d.pq[i] = PagedSeqArg{seqs[i].pages, len, V, npg, K, 0};
    const int64_t last = len - (int64_t)(npg - 1) * ptok;  // keys in the last page
    const int nb_last = (int)((last + kBlk - 1) / kBlk);
    V += (npg - 1) * pstride + (nb_last > 0 ? nb_last : 1);
    vend[i] = V;
    K += npg;
  }
  int nwg = (V + 3) / 4;
  if (nwg > kMainWGs) nwg = kMainWGs;
  if (nwg < 1) nwg = 1;
  const int vq = V / nwg, vr = V % nwg;
  auto wg_of = [&](int x) {
    const int big = vr * (vq + 1);
    return x < big ? x / (vq + 1) : vr + (x - big) / vq;
  };
  for (int i = 0; i < nseq; ++i) {
    c.wg0[i] = wg_of(d.pq[i].vstart) + d.pq[i].kfirst;
    c.wg1[i] = wg_of(vend[i] - 1) + d.pq[i].kfirst + d.pq[i].npg;
  }
  const int nslots = nwg + K;
  d.nseg = nseq;
  d.nwg = nwg;
  d.vq = vq;
  d.vr = vr;
  d.rs_t = rs_t;
  d.rs_h = rs_h;
  d.sl2 = scale * kLog2e;
  d.q = q;
  d.k_new = k_new;
  d.v_new = v_new;
  d.nnew = fused ? nseq : 0;
  d.ncomb = 0;  // several output rows: the separate combine kernel
  d.words = nullptr;
  d.out = out;
  d.prep = DecodePrep{};
  d.q_out = nullptr;
  d.kplane = pool.k;
  d.vplane = pool.v;
  d.page_bytes = pool.page_bytes;
  d.page_lg = pool.page_lg;
  d.pstride = pstride;
  d.nsegs = K;
  const size_t part_floats = (size_t)nslots * 16 * kPartRow, ml_floats = (size_t)nslots * 16 * 2;
  const size_t dq_floats = fused ? (size_t)nseq * 4 * 256 : 0;
  int rc = ws.reserve((part_floats + ml_floats + dq_floats) * sizeof(float));
  if (rc) return rc;
  d.part = static_cast<float *>(ws.ptr);
  d.ml = reinterpret_cast<float2 *>(d.part + part_floats);
  d.dq = fused ? d.part + part_floats + ml_floats : nullptr;
  rc = device_status_word(&d.status);
  if (rc) return rc;
  hipLaunchKernelGGL((q4k_decode_kernel<false, 0>), dim3((unsigned)nwg), dim3(kThreads), 0, s,
                     nullptr, nullptr, q, nullptr, k_new, decode_strides(rs_t, rs_h), 0, nwg, d);
  PKV_HIP(hipGetLastError());
  c.part = d.part;
  c.ml = d.ml;
  c.q = q;
  c.dq = d.dq;
  c.out = out;
  c.sl2 = d.sl2;
  if (const int rc_ = launch_combine(c, nseq, s)) return rc_;
  return PKV_OK;
}

}  // namespace pkv
