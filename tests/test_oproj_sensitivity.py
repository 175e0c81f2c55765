"""The batched o_proj checks can fail for the mistakes its fp16 operands invite. On the CPU,
with the GPU test's data (random Q4K/Q6K rows, N(0,1) activations, 4096 inputs), the
float64 product is compared with the same product computed the way a broken kernel would:
activations rounded to fp16 after the per-token power-of-two scale (the lo halves dropped),
or Q6K weights whose scale is rounded into fp16 with the code ((q - 32) * sc not split).
The RMS-relative bound of the GPU test (2e-5) rejects both, while the oracle tolerance
(2e-3 absolute + 1e-3 relative) alone passes the dropped lo halves. No GPU and no library
code: this checks the checks."""
import numpy as np

import oracle as orc
from kquant_blocks import W_Q4K, W_Q6K, random_weight_bytes

BOUND = 2e-5


def rms_rel_err(got, ref):
    return np.abs(got - ref).max() / np.sqrt((ref ** 2).mean())


def setup(w_type, seed=5):
    rng = np.random.default_rng(seed)
    b, in_dim, out_dim = 16, 4096, 256
    wb = random_weight_bytes(rng, w_type, out_dim, in_dim, d_scale=1e-4)
    wdq = orc.dequantize_weight(wb, w_type, out_dim * in_dim).reshape(out_dim, in_dim)
    x = rng.standard_normal((b, in_dim)).astype(np.float32)
    return wb, wdq.astype(np.float64), x


def scaled(x):
    """x * 2^e per row, max |.| in [2^14, 2^15), and 2^-e"""
    e = 15 - np.frexp(np.abs(x).max(axis=1))[1]
    return np.ldexp(x, e[:, None]), np.ldexp(1.0, -e)


def test_hi_lo_split_passes_and_hi_only_fails():
    _, wdq, x = setup(W_Q4K)
    ref = x.astype(np.float64) @ wdq.T
    xs, inv = scaled(x)
    hi = xs.astype(np.float16).astype(np.float64)
    lo = (xs - hi.astype(np.float32)).astype(np.float16).astype(np.float64)
    good = ((hi + lo) @ wdq.T) * inv[:, None]
    bad = (hi @ wdq.T) * inv[:, None]
    assert rms_rel_err(good, ref) < BOUND / 10
    assert rms_rel_err(bad, ref) > 2 * BOUND
    np.testing.assert_allclose(bad, ref, atol=2e-3, rtol=1e-3)  # the loose bound passes it


def test_unsplit_q6k_scale_fails():
    wb, wdq, x = setup(W_Q6K, seed=6)
    ref = x.astype(np.float64) @ wdq.T
    blk = wb.reshape(-1, 210)
    d = blk[:, 208:210].copy().view(np.float16).astype(np.float64)[:, 0]
    sc = blk[:, 192:208].view(np.int8).astype(np.float64)  # [blocks, 16]
    unit = blk.copy()  # the same codes with d = 1 and every scale 1 decode to q - 32
    unit[:, 192:208] = 1
    unit[:, 208:210] = np.array([1.0], np.float16).view(np.uint8)
    q = orc.dequantize_weight(unit.reshape(-1), W_Q6K, wdq.size).reshape(-1, 256)
    prod = np.repeat(sc, 16, axis=1) * q                                  # (q - 32) sc
    prod16 = prod.astype(np.float16).astype(np.float64)                   # rounded to fp16
    assert np.any(prod16 != prod)
    w_bad = (d[:, None] * prod16).reshape(wdq.shape)
    assert rms_rel_err(x.astype(np.float64) @ w_bad.T, ref) > 2 * BOUND
