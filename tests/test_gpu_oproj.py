"""GPU parity of the gated output projection (pkv_gated_oproj_q4k, pkv_gated_oproj; the step
after the attention, qwen3_next.rs:2657-2680) with a Q4K, Q5K, Q6K or Q8_0 wo against the
CPU oracle's f32 dequantize-then-dot on the same seeded inputs, within 2e-3 absolute +
1e-3 relative. The reference's QMatMul lives in the absent candle fork, so its own
rounding (it may quantize the activations first) is not the bar; the GGUF weight bytes
are shared. Q5K/Q6K/Q8_0 weights are random valid blocks (tests/kquant_blocks.py)."""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-3
Q4K = 4
W_Q8_0, W_Q4K, W_Q5K, W_Q6K = 8, 12, 13, 14


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def pk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import paramecia_amd
    paramecia_amd.lib()
    return paramecia_amd


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


# batches below 4 take one output row per wave, from 4 on two (both kernel forms)
@pytest.mark.parametrize("b,in_dim,out_dim,gated", [(1, 4096, 2048, True), (3, 4096, 100, True),
                                                    (2, 8192, 64, True), (2, 4096, 40, False),
                                                    (5, 4096, 72, True), (4, 8192, 20, True)])
def test_matches_oracle(pk, orc, b, in_dim, out_dim, gated):
    say(f"oproj b={b} in={in_dim} out={out_dim} gated={gated}")
    rng = np.random.default_rng(in_dim + out_dim + b)
    w = (rng.standard_normal((out_dim, in_dim)) * 0.05).astype(np.float32)
    wb = orc.quantize(w.reshape(-1), Q4K)
    x = rng.standard_normal((b, in_dim)).astype(np.float32)
    g = rng.standard_normal((b, in_dim)).astype(np.float32) if gated else None
    out = pk.gated_o_proj(dev(x[:, None]), dev(g[:, None]) if gated else None, dev(wb), out_dim)
    assert tuple(out.shape) == (b, 1, out_dim)
    ref = orc.gated_oproj_q4k(x, g, wb, out_dim)
    np.testing.assert_allclose(host(out)[:, 0], ref, atol=ATOL, rtol=RTOL)


def test_rejects_unsupported_width(pk):
    from paramecia_amd._lib import lib, ERR_UNSUPPORTED
    say("oproj: argument checks")
    x = torch.zeros((1, 1024), device="cuda")
    w = torch.zeros(8 * 4 * 144, dtype=torch.uint8, device="cuda")
    out = torch.zeros((1, 8), device="cuda")
    assert lib().pkv_gated_oproj_q4k(x.data_ptr(), None, w.data_ptr(), out.data_ptr(), 1, 1024, 8,
                                     torch.cuda.current_stream().cuda_stream) == ERR_UNSUPPORTED


# every weight type through pkv_gated_oproj: both row forms (batch < 4, >= 4), both input
# widths, a ragged row tail (out_dim not a multiple of the 4 or 8 rows of a workgroup) and
# no gate
SHAPES = [(1, 4096, 2048, True), (3, 4096, 100, True), (2, 8192, 64, True),
          (2, 4096, 42, False), (5, 4096, 70, True), (4, 8192, 22, True)]


@pytest.mark.parametrize("w_type", [W_Q4K, W_Q5K, W_Q6K, W_Q8_0])
@pytest.mark.parametrize("b,in_dim,out_dim,gated", SHAPES)
def test_weight_types_match_oracle(pk, orc, w_type, b, in_dim, out_dim, gated):
    from kquant_blocks import random_weight_bytes
    say(f"oproj w_type={w_type} b={b} in={in_dim} out={out_dim} gated={gated}")
    rng = np.random.default_rng(1000 * w_type + in_dim + out_dim + b)
    wb = random_weight_bytes(rng, w_type, out_dim, in_dim, d_scale=1e-4)
    x = rng.standard_normal((b, in_dim)).astype(np.float32)
    g = rng.standard_normal((b, in_dim)).astype(np.float32) if gated else None
    out = pk.gated_o_proj(dev(x[:, None]), dev(g[:, None]) if gated else None, dev(wb), out_dim,
                          w_type=w_type)
    ref = orc.gated_oproj(x, g, wb, w_type, out_dim)
    assert np.abs(ref).max() > 0.1  # the weights are not degenerate
    np.testing.assert_allclose(host(out)[:, 0], ref, atol=ATOL, rtol=RTOL)


def test_generic_entry_checks(pk):
    from paramecia_amd._lib import lib, ERR_UNSUPPORTED
    say("oproj: generic entry argument checks")
    x = torch.zeros((1, 4096), device="cuda")
    w = torch.zeros(8 * 16 * 210, dtype=torch.uint8, device="cuda")
    out = torch.zeros((1, 8), device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    assert lib().pkv_gated_oproj(x.data_ptr(), None, w.data_ptr(), 2, out.data_ptr(), 1, 4096, 8,
                                 s) == ERR_UNSUPPORTED  # Q4_1: no kernel
    assert lib().pkv_gated_oproj(x.data_ptr(), None, w.data_ptr(), W_Q6K, out.data_ptr(), 1, 2048,
                                 8, s) == ERR_UNSUPPORTED
    with pytest.raises(pk.KvCacheError):
        pk.gated_o_proj(x[:, None], None, w[:-1], 8, w_type=W_Q6K)


# ---- the batched MFMA form (from 8 tokens on, Q4K/Q5K/Q6K): fp16 hi/lo activations and
# exact scaled weight codes. Besides the oracle's tolerance, the error relative to the
# outputs' RMS must stay below 2e-5: dropping the lo halves (fp16 activations only) gives
# about 2.4e-4, a wrong scale or code far more.
def rms_rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    return np.abs(np.asarray(got, np.float64) - ref).max() / np.sqrt((ref ** 2).mean())


BATCHED = [(8, 4096, 256, True), (33, 4096, 300, True), (40, 8192, 264, False),
           (96, 4096, 520, True), (7, 4096, 64, True)]


@pytest.mark.parametrize("w_type", [W_Q4K, W_Q5K, W_Q6K])
@pytest.mark.parametrize("b,in_dim,out_dim,gated", BATCHED)
def test_batched_form_matches_oracle(pk, orc, w_type, b, in_dim, out_dim, gated):
    from kquant_blocks import random_weight_bytes
    say(f"oproj batched w_type={w_type} b={b} in={in_dim} out={out_dim} gated={gated}")
    rng = np.random.default_rng(3000 * w_type + in_dim + out_dim + b)
    wb = random_weight_bytes(rng, w_type, out_dim, in_dim, d_scale=1e-4)
    x = rng.standard_normal((b, in_dim)).astype(np.float32)
    g = rng.standard_normal((b, in_dim)).astype(np.float32) if gated else None
    out = host(pk.gated_o_proj(dev(x), dev(g) if gated else None, dev(wb), out_dim,
                               w_type=w_type))
    ref = orc.gated_oproj(x, g, wb, w_type, out_dim)
    np.testing.assert_allclose(out, ref, atol=ATOL, rtol=RTOL)
    assert rms_rel_err(out, ref) < 2e-5


def test_batched_form_token_scales(pk, orc):
    """Per-token power-of-two scaling: rows of 1e-30, 1e4 and 0 magnitudes beside N(0, 1)
    rows keep the relative accuracy of each row; the zero row gives exact zeros."""
    from kquant_blocks import random_weight_bytes
    say("oproj batched: token scales")
    rng = np.random.default_rng(77)
    b, in_dim, out_dim = 12, 4096, 96
    wb = random_weight_bytes(rng, W_Q4K, out_dim, in_dim, d_scale=1e-4)
    x = rng.standard_normal((b, in_dim)).astype(np.float32)
    x[1] *= np.float32(1e-30)
    x[2] *= np.float32(1e4)
    x[3] = 0.0
    out = host(pk.gated_o_proj(dev(x), None, dev(wb), out_dim, w_type=W_Q4K))
    ref = orc.gated_oproj(x, None, wb, W_Q4K, out_dim)
    assert np.all(out[3] == 0.0)
    for r in (0, 1, 2, 4):
        assert rms_rel_err(out[r], ref[r]) < 2e-5, r


@pytest.mark.parametrize("w_type", [W_Q4K, W_Q6K])
def test_batched_form_prefill_chunk(pk, orc, w_type):
    """The config-2 prefill chunk at full size: 512 tokens through a 4096 -> 2048 wo, against
    a float64 product over the oracle's dequantized rows."""
    from kquant_blocks import random_weight_bytes
    say(f"oproj batched: 512-token chunk w_type={w_type}")
    rng = np.random.default_rng(512 + w_type)
    b, in_dim, out_dim = 512, 4096, 2048
    wb = random_weight_bytes(rng, w_type, out_dim, in_dim, d_scale=1e-4)
    x = rng.standard_normal((b, in_dim)).astype(np.float32)
    g = rng.standard_normal((b, in_dim)).astype(np.float32)
    out = host(pk.gated_o_proj(dev(x[None]), dev(g[None]), dev(wb), out_dim, w_type=w_type))[0]
    wdq = orc.dequantize_weight(wb, w_type, out_dim * in_dim).reshape(out_dim, in_dim)
    y = x.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))
    ref = y @ wdq.astype(np.float64).T
    assert rms_rel_err(out, ref) < 2e-5
