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

// Paged decode: every page run is a segment; the combine merges all partials of a
// sequence (its segments are consecutive). Up to kMaxSegs segments travel in the kernel
// arguments (also under stream capture), each page with the same number of workgroups
// (wps, fixed mode: workgroup w serves segment w / wps). More pages go to a device table
// staged through the workspace and are split stream-K: the pages' blocks on one virtual
// line with a gap before every page after the first (the cost of one more pass), 256
// workgroups with equal ranges, one partial per piece, the pieces of a sequence in
// consecutive slots (the per-workgroup first segment and first slot travel in the
// table too).
int launch_paged_decode_q4k(const PagedSeg *segs, int nseg, int nseq, int page_tokens,
                            const float *q, float *out, int64_t rs_t, int64_t rs_h,
                            float scale, void *stage, Workspace &ws, hipStream_t s,
                            const float *k_new, const float *v_new, const NewRow *rows) {
  // the staging buffer holds nseg * kPagedSegBytes + kPagedStageExtra bytes
  static_assert(sizeof(DecodeSeg) <= kPagedSegBytes, "segment table entry size");
  static_assert(kMainWGs * sizeof(int2) + kMaxPagedSeqs * sizeof(NewRow) <= kPagedStageExtra,
                "workgroup and new-row table size");
  const bool fused = k_new != nullptr;
  if (fused && (v_new == nullptr || rows == nullptr))
    return set_error(PKV_ERR_ARG, "paged decode: fused step without its new rows");
  static_assert(kPagedArgSegs == kMaxSegs, "kernel-argument segment count");
  if (nseq < 1 || nseq > kMaxPagedSeqs || nseg < nseq || page_tokens % kBlk != 0)
    return set_error(PKV_ERR_ARG, "paged decode: bad segment plan");
  if (!decode_rows_fit(page_tokens, rs_t)) return PKV_ERR_UNSUPPORTED;
  if (nseg > (1 << 20)) return set_error(PKV_ERR_ARG, "paged decode: too many pages");
  const bool stream = fused || nseg > kMaxSegs;
  std::vector<DecodeSeg> tab((size_t)nseg);
  int qprev = -1;
  int V = 0;
  for (int i = 0; i < nseg; ++i) {
    DecodeSeg &d = tab[(size_t)i];
    if (segs[i].qi < qprev || segs[i].qi >= nseq || segs[i].len < 0 || segs[i].len > page_tokens)
      return set_error(PKV_ERR_ARG, "paged decode: segments out of order");
    if (segs[i].qi > qprev + 1) return set_error(PKV_ERR_ARG, "paged decode: a sequence has no page");
    qprev = segs[i].qi;
    d.k = segs[i].k;
    d.v = segs[i].v;
    d.seq_k = segs[i].len;
    d.t_new = 0;
    d.nblk = (int)((segs[i].len + kBlk - 1) / kBlk);
    d.qi = segs[i].qi;
    if (i > 0) V += kPieceGap;
    d.voff = V;
    V += d.nblk > 0 ? d.nblk : 1;
  }
  if (qprev != nseq - 1) return set_error(PKV_ERR_ARG, "paged decode: a sequence has no page");
  DecodeArgsT<kMaxSegs> d;
  CombineArgs c;
  int nwg, nslots;
  std::vector<int2> wt;
  if (!stream) {
    // blocks per workgroup: the multiple of 4 that minimises the estimated makespan
    // (rounds of 256 workgroups x (bpw / 4 blocks per wave + ~1.3 blocks of set-up))
    const int pblk = page_tokens / kBlk;
    int bpw = 4;
    double best = 1e30;
    for (int cand = 4; cand <= ((pblk + 3) / 4) * 4 && cand <= 64; cand += 4) {
      const int64_t w = (int64_t)nseg * ((pblk + cand - 1) / cand);
      const double cost = (double)((w + kMainWGs - 1) / kMainWGs) * (cand / 4.0 + 1.3);
      if (cost < best) {
        best = cost;
        bpw = cand;
      }
    }
    const int wps = (pblk + bpw - 1) / bpw;
    nwg = nseg * wps;
    nslots = nwg;
    for (int i = 0; i < nseg; ++i) {
      tab[(size_t)i].wg0 = i * wps;
      const int qi = tab[(size_t)i].qi;
      if (i == 0 || tab[(size_t)i - 1].qi != qi) c.wg0[qi] = i * wps;
      c.wg1[qi] = (i + 1) * wps;
    }
    d.bpw = bpw;
    d.wps = wps;
    d.vq = d.vr = 0;
  } else {
    nwg = (V + 3) / 4;
    if (nwg > kMainWGs) nwg = kMainWGs;
    const int vq = V / nwg, vr = V % nwg;
    wt.resize((size_t)nwg);
    for (int q2 = 0; q2 < nseq; ++q2) c.wg0[q2] = -1;
    int slot = 0, sfirst = 0;
    for (int w = 0; w < nwg; ++w) {
      const int V0 = w * vq + (w < vr ? w : vr), V1 = V0 + vq + (w < vr ? 1 : 0);
      auto vend = [&](int i) {
        return tab[(size_t)i].voff + (tab[(size_t)i].nblk > 0 ? tab[(size_t)i].nblk : 1);
      };
      while (sfirst < nseg && vend(sfirst) <= V0) ++sfirst;
      wt[(size_t)w] = int2{sfirst, slot};
      for (int i = sfirst; i < nseg && tab[(size_t)i].voff < V1; ++i) {
        const int qi = tab[(size_t)i].qi;
        if (c.wg0[qi] < 0) c.wg0[qi] = slot;
        c.wg1[qi] = ++slot;
      }
    }
    nslots = slot;
    for (int i = 0; i < nseg; ++i) tab[(size_t)i].wg0 = 0;  // no prepared q on this path
    d.bpw = 0;
    d.wps = 0;
    d.vq = vq;
    d.vr = vr;
  }
  d.nseg = nseg;
  d.nwg = nwg;
  d.rs_t = rs_t;
  d.rs_h = rs_h;
  d.sl2 = scale * kLog2e;
  d.q = q;
  d.k_new = k_new;
  d.v_new = v_new;
  d.nnew = fused ? nseq : 0;
  d.prep = DecodePrep{};
  d.q_out = nullptr;
  const size_t part_floats = (size_t)nslots * 16 * kPartRow, ml_floats = (size_t)nslots * 16 * 2;
  const size_t dq_floats = fused ? (size_t)nseq * 4 * 256 : 0;
  const size_t tab_off = (part_floats + ml_floats + dq_floats) * sizeof(float);
  const size_t seg_bytes = stream ? (size_t)nseg * sizeof(DecodeSeg) : 0;
  const size_t wt_bytes = stream ? (size_t)nwg * sizeof(int2) : 0;
  const size_t row_bytes_ = fused ? (size_t)nseq * sizeof(NewRow) : 0;
  const size_t tab_bytes = seg_bytes + wt_bytes + row_bytes_;
  int rc = ws.reserve(tab_off + tab_bytes);
  if (rc) return rc;
  d.part = static_cast<float *>(ws.ptr);
  d.ml = reinterpret_cast<float2 *>(d.part + part_floats);
  d.dq = fused ? d.part + part_floats + ml_floats : nullptr;
  rc = device_status_word(&d.status);
  if (rc) return rc;
  d.newrows = nullptr;
  if (!stream) {
    for (int i = 0; i < nseg; ++i) d.seg[i] = tab[(size_t)i];
    d.dseg = nullptr;
    d.wtab = nullptr;
  } else {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    PKV_HIP(hipStreamIsCapturing(s, &cap));
    if (cap != hipStreamCaptureStatusNone)
      return set_error(PKV_ERR_UNSUPPORTED,
                       "paged decode over more than 32 pages cannot be captured in a graph");
    if (stage == nullptr) return set_error(PKV_ERR_ARG, "paged decode: no staging buffer");
    memcpy(stage, tab.data(), seg_bytes);
    memcpy(static_cast<uint8_t *>(stage) + seg_bytes, wt.data(), wt_bytes);
    if (fused) memcpy(static_cast<uint8_t *>(stage) + seg_bytes + wt_bytes, rows, row_bytes_);
    uint8_t *dtab = static_cast<uint8_t *>(ws.ptr) + tab_off;
    PKV_HIP(hipMemcpyAsync(dtab, stage, tab_bytes, hipMemcpyHostToDevice, s));
    d.dseg = reinterpret_cast<DecodeSeg *>(dtab);
    d.wtab = reinterpret_cast<const int2 *>(dtab + seg_bytes);
    if (fused) d.newrows = reinterpret_cast<const NewRow *>(dtab + seg_bytes + wt_bytes);
  }
  hipLaunchKernelGGL((q4k_decode_kernel<false, kMaxSegs>), dim3((unsigned)nwg), dim3(kThreads), 0,
                     s, d);
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
