"""Pins of the oracle's gated output projection (orc_gated_oproj_q4k; qwen3_next.rs:2657-2680:
sigmoid gate, then the Q4K wo QMatMul): a float64 numpy restatement over the oracle's
pinned Q4K dequantizer, and closed forms of the gate. A transposed weight, a dropped
gate or a wrong sub-block scale fails one of them."""
import numpy as np

import oracle as orc

Q4K = 4


def weights(rng, out_dim, in_dim):
    w = (rng.standard_normal((out_dim, in_dim)) * 0.05).astype(np.float32)
    wb = orc.quantize(w.reshape(-1), Q4K)
    wdq = orc.dequantize(wb, Q4K, out_dim * in_dim).reshape(out_dim, in_dim)
    return wb, wdq


def test_matches_float64_restatement():
    rng = np.random.default_rng(11)
    b, in_dim, out_dim = 2, 4096, 48
    wb, wdq = weights(rng, out_dim, in_dim)
    x = rng.standard_normal((b, in_dim)).astype(np.float32)
    g = rng.standard_normal((b, in_dim)).astype(np.float32)
    y64 = (wdq.astype(np.float64) @ (x.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))).T).T
    np.testing.assert_allclose(orc.gated_oproj_q4k(x, g, wb, out_dim), y64, rtol=1e-4, atol=2e-5)


def test_gate_closed_forms():
    rng = np.random.default_rng(12)
    b, in_dim, out_dim = 1, 4096, 16
    wb, wdq = weights(rng, out_dim, in_dim)
    x = rng.standard_normal((b, in_dim)).astype(np.float32)
    plain = orc.gated_oproj_q4k(x, None, wb, out_dim)
    np.testing.assert_allclose(plain, (wdq.astype(np.float64) @ x[0].astype(np.float64))[None],
                               rtol=1e-4, atol=2e-5)
    open_gate = orc.gated_oproj_q4k(x, np.full_like(x, 100.0), wb, out_dim)
    np.testing.assert_array_equal(open_gate, plain)  # sigmoid(100) rounds to 1
    half = orc.gated_oproj_q4k(x, np.zeros_like(x), wb, out_dim)
    np.testing.assert_array_equal(half, plain * np.float32(0.5))  # exact power-of-two scaling
    shut = orc.gated_oproj_q4k(x, np.full_like(x, -100.0), wb, out_dim)
    assert np.abs(shut).max() < 1e-30
