"""GPU tests of the MFMA prefill-chunk paths (Q4K and Q8_0, 16 q heads / 2 KV heads /
head_dim 256, l > 1): causal masks with and without a q_offset, chunk lengths around the
16-position tile, batch > 1, key splits merged and unsplit, outlier channels, and the
full prefill-chunk configuration (512 queries over 16896 keys) against the CPU oracle's
float64 attention over the dequantized rows (assert_attn_close: 2e-3 absolute + 1e-3
relative per element, 2e-5 relative L2, 1e-4 of the largest output); the appended
chunk's bytes must be bit-exact."""
import sys

import numpy as np
import pytest

from attn_checks import assert_attn_close

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

Q8_0, Q4K = 3, 4
QUANTS = [pytest.param(Q4K, id="q4k"), pytest.param(Q8_0, id="q8_0")]
ATOL, RTOL = 2e-3, 1e-3


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


def run_prefill(pk, orc, S, L, B=1, causal=True, seed=0, chans=None, quant=Q4K):
    """S cached keys, then a chunk of L tokens appended; its L queries attend over all
    S + L keys (causal: query i sees keys j <= S + i)."""
    rng = np.random.default_rng(seed)
    g = pk.PreallocatedQuantizedKvCache(B, 2, S + L, 256, pk.KvCacheQuantization(quant))
    c = orc.Cache(quant, B, 2, 256, S + L)
    k = rng.standard_normal((B, 2, S + L, 256)).astype(np.float32)
    v = rng.standard_normal((B, 2, S + L, 256)).astype(np.float32)
    q = rng.standard_normal((B, L, 16, 256)).astype(np.float32)
    if chans is not None:
        for x in (k, v):
            x[..., chans] *= 20.0
    if S > 0:
        g.append_quantized(dev(k[:, :, :S]), dev(v[:, :, :S]))
    g.append_quantized(dev(k[:, :, S:]), dev(v[:, :, S:]), offset=S)
    assert c.append(k, v) == 0
    out = g.attend(dev(q), 1 / 16, S, causal)
    ref = c.attend(q, 1 / 16, S, causal, mode="f64")
    got = host(out)
    assert_attn_close(got, ref)
    gk, gv = g.raw_bytes()
    ok, ov = c.valid_bytes()
    assert np.array_equal(host(gk), ok) and np.array_equal(host(gv), ov)
    return np.abs(got - ref).max()


@pytest.mark.parametrize("quant", QUANTS)
@pytest.mark.parametrize("S,L", [(0, 2), (0, 16), (0, 17), (5, 15), (31, 33), (64, 64),
                                 (1000, 40), (3000, 100), (0, 300)])
def test_prefill_causal(pk, orc, S, L, quant):
    say(f"prefill causal quant={quant} S={S} L={L}")
    run_prefill(pk, orc, S, L, seed=S * 7 + L, quant=quant)


@pytest.mark.parametrize("quant", QUANTS)
@pytest.mark.parametrize("S,L", [(100, 3), (777, 48)])
def test_prefill_noncausal(pk, orc, S, L, quant):
    say(f"prefill non-causal quant={quant} S={S} L={L}")
    run_prefill(pk, orc, S, L, causal=False, seed=S + L + 1, quant=quant)


@pytest.mark.parametrize("quant", QUANTS)
def test_prefill_batch2(pk, orc, quant):
    say(f"prefill batch 2 quant={quant}")
    run_prefill(pk, orc, 500, 37, B=2, seed=11, quant=quant)


@pytest.mark.parametrize("quant", QUANTS)
def test_prefill_unsplit(pk, orc, quant):
    """2048 queries fill 256 workgroups without a key split (no merge kernel)."""
    say(f"prefill unsplit L=2048 quant={quant}")
    run_prefill(pk, orc, 0, 2048, seed=12, quant=quant)


@pytest.mark.parametrize("quant", QUANTS)
def test_prefill_outlier_channels(pk, orc, quant):
    say(f"prefill outlier channels quant={quant}")
    from paramecia_amd import workloads as W
    run_prefill(pk, orc, 4000, 64, seed=13, chans=W.c5_channels(), quant=quant)


@pytest.mark.parametrize("quant", QUANTS)
def test_prefill_full_chunk(pk, orc, quant):
    """The prefill-chunk configuration: 16384 cached tokens, a 512-token chunk appended
    at offset 16384, causal attention of its queries over 16896 keys; seeded data
    generated on the GPU and on the CPU. The Q8_0 case also scales the outlier channels
    by 20 on both sides (a Q8_0 block's scale then comes from its outlier)."""
    from paramecia_amd import workloads as W
    S, C = 16384, 512
    chans = W.c5_channels() if quant == Q8_0 else None
    say(f"full prefill chunk quant={quant}: GPU")
    g = pk.PreallocatedQuantizedKvCache(1, 2, 32768, 256, pk.KvCacheQuantization(quant))
    kb = torch.empty((1, 2, S, 256), device="cuda")
    vb = torch.empty_like(kb)
    pk.fill_normal(kb, W.SEED, W.stream_id(2, W.T_PREFILL_K))
    pk.fill_normal(vb, W.SEED, W.stream_id(2, W.T_PREFILL_V))
    if chans is not None:
        for x in (kb, vb):
            x[..., torch.as_tensor(chans, device="cuda")] *= 20.0
    g.append_quantized(kb, vb)
    del kb, vb
    kc = torch.empty((1, 2, C, 256), device="cuda")
    vc = torch.empty_like(kc)
    qc = torch.empty((1, C, 16, 256), device="cuda")
    pk.fill_normal(kc, W.SEED, W.stream_id(2, W.T_CHUNK_K))
    pk.fill_normal(vc, W.SEED, W.stream_id(2, W.T_CHUNK_V))
    pk.fill_normal(qc, W.SEED, W.stream_id(2, W.T_CHUNK_Q))
    if chans is not None:
        for x in (kc, vc):
            x[..., torch.as_tensor(chans, device="cuda")] *= 20.0
    g.append_quantized(kc, vc, offset=S)
    out = host(g.attend(qc, W.SCALE, S, causal=True))
    gk, gv = (host(x) for x in g.raw_bytes())
    say(f"full prefill chunk quant={quant}: CPU oracle")
    c = orc.Cache(quant, 1, 2, 256, S + C)
    k = orc.normal(2 * S * 256, W.SEED, W.stream_id(2, W.T_PREFILL_K)).reshape(1, 2, S, 256)
    v = orc.normal(2 * S * 256, W.SEED, W.stream_id(2, W.T_PREFILL_V)).reshape(1, 2, S, 256)
    if chans is not None:
        for x in (k, v):
            x[..., chans] *= np.float32(20.0)
    assert c.append(k, v) == 0
    del k, v
    kcn = orc.normal(2 * C * 256, W.SEED, W.stream_id(2, W.T_CHUNK_K)).reshape(1, 2, C, 256)
    vcn = orc.normal(2 * C * 256, W.SEED, W.stream_id(2, W.T_CHUNK_V)).reshape(1, 2, C, 256)
    qcn = orc.normal(C * 16 * 256, W.SEED, W.stream_id(2, W.T_CHUNK_Q)).reshape(1, C, 16, 256)
    if chans is not None:
        for x in (kcn, vcn):
            x[..., chans] *= np.float32(20.0)
    assert c.append(kcn, vcn) == 0
    ok, ov = c.valid_bytes()
    assert np.array_equal(gk, ok), "K bytes differ"
    assert np.array_equal(gv, ov), "V bytes differ"
    ref = c.attend(qcn, W.SCALE, S, True, mode="f64")
    err = np.abs(out - ref)
    say(f"full prefill chunk quant={quant}: max|diff| = {err.max():.3e}")
    assert_attn_close(out, ref)
