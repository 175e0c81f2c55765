"""GPU tests of the MFMA decode path (Q4K, 16 q heads / 2 KV heads / head_dim 256):
block-boundary sizes, batch > 1, outlier channels, and one full-size layer of the
headline configuration (131072 cached tokens) against the CPU oracle."""
import sys

import numpy as np
import pytest

from attn_checks import assert_attn_close

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

Q4K = 4
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


def run_decode(pk, orc, S, B=1, fused=True, seed=0, k_scale=None, chans=None):
    rng = np.random.default_rng(seed)
    g = pk.PreallocatedQuantizedKvCache(B, 2, S + 1, 256, pk.KvCacheQuantization.Q4K)
    c = orc.Cache(Q4K, B, 2, 256, S + 1)
    k = rng.standard_normal((B, 2, S, 256)).astype(np.float32)
    v = rng.standard_normal((B, 2, S, 256)).astype(np.float32)
    q = rng.standard_normal((B, 1, 16, 256)).astype(np.float32)
    kn = rng.standard_normal((B, 2, 1, 256)).astype(np.float32)
    vn = rng.standard_normal((B, 2, 1, 256)).astype(np.float32)
    if chans is not None:
        for x in (k, v, kn, vn):
            x[..., chans] *= 20.0
    if S > 0:
        g.append_quantized(dev(k), dev(v))
        assert c.append(k, v) == 0
    if fused:
        out = g.append_attend(dev(kn), dev(vn), dev(q), 1 / 16)
        assert c.append(kn, vn) == 0
        seq = S + 1
    else:
        out = g.attend(dev(q), 1 / 16, S - 1, True)
        seq = S
    ref = c.attend(q, 1 / 16, seq - 1, True, mode="f64")
    got = host(out)
    assert_attn_close(got, ref)
    gk, gv = g.raw_bytes()
    ok, ov = c.valid_bytes()
    assert np.array_equal(host(gk), ok) and np.array_equal(host(gv), ov)
    assert pk.lib().pkv_device_status() == 0, pk.lib().pkv_last_error()
    return np.abs(got - ref).max()


@pytest.mark.parametrize("S", [0, 1, 2, 31, 32, 33, 95, 96, 97, 128, 129, 255, 1000, 4096, 4127])
def test_decode_fused_boundaries(pk, orc, S):
    say(f"fused decode S={S}")
    run_decode(pk, orc, S, fused=True, seed=S)


@pytest.mark.parametrize("S", [1, 32, 33, 130, 2049])
def test_decode_attend_only(pk, orc, S):
    say(f"attend-only decode S={S}")
    run_decode(pk, orc, S, fused=False, seed=1000 + S)


def test_decode_batch2(pk, orc):
    say("decode batch 2")
    run_decode(pk, orc, 777, B=2, seed=5)


def test_decode_outlier_channels(pk, orc):
    say("decode outlier channels")
    from paramecia_amd import workloads as W
    run_decode(pk, orc, 20000, seed=6, chans=W.c5_channels())


def test_decode_full_size_layer(pk, orc):
    """One layer of the headline workload: seeded data generated on the GPU and on the
    CPU must give the same Q4K bytes (131072 tokens x 4 rows), and the fused decode
    step must match the oracle's f32 attention over 131073 keys."""
    from paramecia_amd import workloads as W
    S = 131072
    say("full-size layer: generate + quantize on GPU")
    kbuf = torch.empty((1, 2, S, 256), dtype=torch.float32, device="cuda")
    vbuf = torch.empty_like(kbuf)
    pk.fill_normal(kbuf, W.SEED, W.stream_id(3, W.T_PREFILL_K, 0))
    pk.fill_normal(vbuf, W.SEED, W.stream_id(3, W.T_PREFILL_V, 0))
    g = pk.PreallocatedQuantizedKvCache(1, 2, S + 1, 256, pk.KvCacheQuantization.Q4K)
    g.append_quantized(kbuf, vbuf)
    q = torch.empty((1, 1, 16, 256), dtype=torch.float32, device="cuda")
    kn = torch.empty((1, 2, 1, 256), dtype=torch.float32, device="cuda")
    vn = torch.empty_like(kn)
    pk.fill_normal(q, W.SEED, W.stream_id(3, W.T_Q, 0))
    pk.fill_normal(kn, W.SEED, W.stream_id(3, W.T_NEW_K, 0))
    pk.fill_normal(vn, W.SEED, W.stream_id(3, W.T_NEW_V, 0))
    out = host(g.append_attend(kn, vn, q, W.SCALE, offset=S))
    gk, gv = (host(x) for x in g.raw_bytes())
    del kbuf, vbuf
    say("full-size layer: CPU oracle quantize + attend")
    c = orc.Cache(Q4K, 1, 2, 256, S + 1)
    k = orc.normal(2 * S * 256, W.SEED, W.stream_id(3, W.T_PREFILL_K, 0)).reshape(1, 2, S, 256)
    v = orc.normal(2 * S * 256, W.SEED, W.stream_id(3, W.T_PREFILL_V, 0)).reshape(1, 2, S, 256)
    assert c.append(k, v) == 0
    del k, v
    knp = orc.normal(512, W.SEED, W.stream_id(3, W.T_NEW_K, 0)).reshape(1, 2, 1, 256)
    vnp = orc.normal(512, W.SEED, W.stream_id(3, W.T_NEW_V, 0)).reshape(1, 2, 1, 256)
    qnp = orc.normal(4096, W.SEED, W.stream_id(3, W.T_Q, 0)).reshape(1, 1, 16, 256)
    assert c.append(knp, vnp) == 0
    ok, ov = c.valid_bytes()
    assert np.array_equal(gk, ok), "K bytes differ"
    assert np.array_equal(gv, ov), "V bytes differ"
    ref = c.attend(qnp, W.SCALE, S, True, mode="f64")
    err = np.abs(out - ref)
    say(f"full-size layer: max|diff| = {err.max():.3e}")
    assert_attn_close(out, ref)


def run_batched(pk, orc, lens, seed, chans=None):
    """One batched decode step over len(lens) caches of different lengths: each gets a
    new token appended (bit-exact bytes) and its query attends over all its keys."""
    rng = np.random.default_rng(seed)
    caches, oracles = [], []
    for S in lens:
        g = pk.PreallocatedQuantizedKvCache(1, 2, S + 1, 256, pk.KvCacheQuantization.Q4K)
        c = orc.Cache(Q4K, 1, 2, 256, S + 1)
        if S > 0:
            k = rng.standard_normal((1, 2, S, 256)).astype(np.float32)
            v = rng.standard_normal((1, 2, S, 256)).astype(np.float32)
            if chans is not None:
                k[..., chans] *= 20.0
                v[..., chans] *= 20.0
            g.append_quantized(dev(k), dev(v))
            assert c.append(k, v) == 0
        caches.append(g)
        oracles.append(c)
    n = len(lens)
    kn = rng.standard_normal((n, 2, 256)).astype(np.float32)
    vn = rng.standard_normal((n, 2, 256)).astype(np.float32)
    if chans is not None:
        kn[..., chans] *= 20.0
        vn[..., chans] *= 20.0
    q = rng.standard_normal((n, 16, 256)).astype(np.float32)
    out = host(pk.append_attend_batched(caches, dev(kn), dev(vn), dev(q), 1 / 16))
    worst = 0.0
    for i, (g, c, S) in enumerate(zip(caches, oracles, lens)):
        assert c.append(kn[i][None, :, None], vn[i][None, :, None]) == 0
        ref = c.attend(q[i][None, None], 1 / 16, S, True, mode="f64")[0, 0]
        assert_attn_close(out[i], ref)
        worst = max(worst, float(np.abs(out[i] - ref).max()))
        assert g.seq_len == S + 1
        gk, gv = g.raw_bytes()
        ok, ov = c.valid_bytes()
        assert np.array_equal(host(gk), ok) and np.array_equal(host(gv), ov)
    assert pk.lib().pkv_device_status() == 0, pk.lib().pkv_last_error()
    return worst


def test_batched_varlen_edges(pk, orc):
    """Empty, single-token and block-boundary caches in one launch."""
    say("batched decode, edge lengths")
    run_batched(pk, orc, [0, 1, 31, 32, 33, 127, 128, 129, 1000, 4095], seed=20)


def test_batched_over_segment_limit(pk, orc):
    """More sequences than one launch takes (32): the call splits into launches."""
    say("batched decode, 40 sequences")
    lens = [int(x) for x in np.random.default_rng(21).integers(1, 700, size=40)]
    run_batched(pk, orc, lens, seed=21)


def test_batched_stream_tiny_and_empty(pk, orc):
    """32 sequences of 0-40 keys in one launch: the launch's blocks lie on one line with
    a gap before every sequence, so most workgroups' ranges cross a boundary or fall in a
    gap (no blocks at all), and the 128 new rows outnumber the workgroups."""
    say("batched decode, 32 tiny sequences")
    lens = [int(x) for x in np.random.default_rng(23).integers(0, 41, size=32)]
    lens[:6] = [0, 0, 1, 31, 32, 33]
    run_batched(pk, orc, lens, seed=23)


def test_batched_stream_long_and_short(pk, orc):
    """One long sequence among short ones: the long one spans most workgroups, the short
    ones share workgroups, so a piece boundary falls inside many workgroups' ranges."""
    say("batched decode, long and short sequences")
    rng = np.random.default_rng(24)
    lens = [20000] + [int(x) for x in rng.integers(1, 300, size=15)] + [4096, 4097, 31, 1, 6000]
    run_batched(pk, orc, lens, seed=24)


def test_batched_outliers_config5_shape(pk, orc):
    """16 sequences of seeded lengths with the config-5 outlier channels (x20), at
    lengths cut to 1/8 of config 5's so the oracle stays fast."""
    say("batched decode, config-5 shape (lengths / 8)")
    from paramecia_amd import workloads as W
    lens = [max(1, S // 8) for S in W.c5_lengths()]
    worst = run_batched(pk, orc, lens, seed=22, chans=W.c5_channels())
    say(f"batched decode, config-5 shape: max|diff| = {worst:.3e}")


# ---- Q8_0 decode (the flash_attn_q8 role): same shape, 272-byte rows
Q8_0 = 3


def run_decode_q8(pk, orc, S, B=1, fused=True, seed=0, chans=None):
    rng = np.random.default_rng(seed)
    g = pk.PreallocatedQuantizedKvCache(B, 2, S + 1, 256, pk.KvCacheQuantization.Q8_0)
    c = orc.Cache(Q8_0, B, 2, 256, S + 1)
    k = rng.standard_normal((B, 2, S, 256)).astype(np.float32)
    v = rng.standard_normal((B, 2, S, 256)).astype(np.float32)
    q = rng.standard_normal((B, 1, 16, 256)).astype(np.float32)
    kn = rng.standard_normal((B, 2, 1, 256)).astype(np.float32)
    vn = rng.standard_normal((B, 2, 1, 256)).astype(np.float32)
    if chans is not None:
        for x in (k, v, kn, vn):
            x[..., chans] *= 20.0
    if S > 0:
        g.append_quantized(dev(k), dev(v))
        assert c.append(k, v) == 0
    if fused:
        out = g.append_attend(dev(kn), dev(vn), dev(q), 1 / 16)
        assert c.append(kn, vn) == 0
        seq = S + 1
    else:
        out = g.attend(dev(q), 1 / 16, S - 1, True)
        seq = S
    ref = c.attend(q, 1 / 16, seq - 1, True, mode="f64")
    got = host(out)
    assert_attn_close(got, ref)
    gk, gv = g.raw_bytes()
    ok, ov = c.valid_bytes()
    assert np.array_equal(host(gk), ok) and np.array_equal(host(gv), ov)
    return np.abs(got - ref).max()


# The MFMA kernel takes caches up to 32768 keys (one 32-key block per workgroup up to
# 8192, two up to 16384, ...: 8223 and 16385 end in a partial block of a workgroup's last
# pass); 32769 and 40000 take the VALU kernel's 32-key chunks.
@pytest.mark.parametrize("S", [0, 1, 15, 16, 17, 31, 32, 33, 511, 512, 513, 4096, 8192, 8193,
                               8223, 16385, 20000, 32768, 32769, 40000])
def test_q8_decode_fused(pk, orc, S):
    say(f"Q8_0 fused decode S={S}")
    run_decode_q8(pk, orc, S, fused=True, seed=300 + S)


def test_q8_decode_outliers_multiblock(pk, orc):
    """Outlier channels (x20) over 20000 keys: three 32-key blocks per MFMA workgroup, so
    the running max rises between blocks and the sums are rescaled."""
    say("Q8_0 decode outlier channels, 20000 keys")
    from paramecia_amd import workloads as W
    run_decode_q8(pk, orc, 20000, seed=501, chans=W.c5_channels())


@pytest.mark.parametrize("S", [1, 64, 4097])
def test_q8_decode_attend_only(pk, orc, S):
    say(f"Q8_0 attend-only decode S={S}")
    run_decode_q8(pk, orc, S, fused=False, seed=400 + S)


def test_q8_decode_batch2_outliers(pk, orc):
    say("Q8_0 decode batch 2, outlier channels")
    from paramecia_amd import workloads as W
    run_decode_q8(pk, orc, 3000, B=2, seed=500, chans=W.c5_channels())


def test_q8_batched_varlen(pk, orc):
    say("Q8_0 batched decode, varied lengths")
    rng = np.random.default_rng(23)
    lens = [0, 1, 33, 700, 2500]
    caches, oracles = [], []
    for S in lens:
        g = pk.PreallocatedQuantizedKvCache(1, 2, S + 1, 256, pk.KvCacheQuantization.Q8_0)
        c = orc.Cache(Q8_0, 1, 2, 256, S + 1)
        if S > 0:
            k = rng.standard_normal((1, 2, S, 256)).astype(np.float32)
            v = rng.standard_normal((1, 2, S, 256)).astype(np.float32)
            g.append_quantized(dev(k), dev(v))
            assert c.append(k, v) == 0
        caches.append(g)
        oracles.append(c)
    n = len(lens)
    kn = rng.standard_normal((n, 2, 256)).astype(np.float32)
    vn = rng.standard_normal((n, 2, 256)).astype(np.float32)
    q = rng.standard_normal((n, 16, 256)).astype(np.float32)
    out = host(pk.append_attend_batched(caches, dev(kn), dev(vn), dev(q), 1 / 16))
    for i, (g, c, S) in enumerate(zip(caches, oracles, lens)):
        assert c.append(kn[i][None, :, None], vn[i][None, :, None]) == 0
        ref = c.attend(q[i][None, None], 1 / 16, S, True, mode="f64")[0, 0]
        assert_attn_close(out[i], ref)
        gk, gv = g.raw_bytes()
        ok, ov = c.valid_bytes()
        assert np.array_equal(host(gk), ok) and np.array_equal(host(gv), ov)


def test_inlaunch_combine_replays_and_mixed_sizes(pk, orc):
    """One-row decodes over 256 workgroups merge their partials inside the decode launch,
    polling words that carry the launch parity (a per-handle region every such launch
    rewrites). On one handle: eager fused steps, a captured step replayed three times with
    other eager steps (which flip the parity) in between, and shorter decodes that take
    the separate combine in between: every output equals the first eager output bit for
    bit, or the oracle's for a different input."""
    say("in-launch combine: graph replays, eager steps and short decodes interleaved")
    S, Sshort = 40000, 3000
    rng = np.random.default_rng(77)
    g = pk.PreallocatedQuantizedKvCache(1, 2, S + 1, 256, pk.KvCacheQuantization.Q4K)
    c = orc.Cache(Q4K, 1, 2, 256, S + 1)
    k = rng.standard_normal((1, 2, S, 256)).astype(np.float32)
    v = rng.standard_normal((1, 2, S, 256)).astype(np.float32)
    g.append_quantized(dev(k), dev(v))
    assert c.append(k, v) == 0
    kn = rng.standard_normal((1, 2, 1, 256)).astype(np.float32)
    vn = rng.standard_normal((1, 2, 1, 256)).astype(np.float32)
    q = rng.standard_normal((1, 1, 16, 256)).astype(np.float32)
    q2 = rng.standard_normal((1, 1, 16, 256)).astype(np.float32)
    dkn, dvn, dq, dq2 = dev(kn), dev(vn), dev(q), dev(q2)
    ref = host(g.append_attend(dkn, dvn, dq, 1 / 16, offset=S))
    assert c.append(kn, vn) == 0
    assert_attn_close(ref, c.attend(q, 1 / 16, S, True, mode="f64"), what="eager fused step")
    ref2 = c.attend(q2, 1 / 16, S, True, mode="f64")
    cs = orc.Cache(Q4K, 1, 2, 256, Sshort)
    cs.load_bytes(*c.valid_bytes(), Sshort)
    ref_short = cs.attend(q, 1 / 16, Sshort - 1, True, mode="f64")
    outs = [None]

    def step():
        outs[0] = g.append_attend(dkn, dvn, dq, 1 / 16, offset=S)

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    got = outs[0]
    for i in range(3):
        for j in range(i + 1):  # eager fused steps with another query: the parity moves on
            assert_attn_close(host(g.append_attend(dkn, dvn, dq2, 1 / 16, offset=S)), ref2,
                              what=f"eager step {i}.{j}")
        g.set_len(Sshort)  # a shorter decode: fewer workgroups, the separate combine
        assert_attn_close(host(g.attend(dq, 1 / 16, Sshort - 1)), ref_short, what=f"short {i}")
        g.set_len(S + 1)
        graph.replay()
        assert np.array_equal(host(got), ref), f"replay {i}"
        assert np.array_equal(host(g.append_attend(dkn, dvn, dq, 1 / 16, offset=S)), ref), f"eager {i}"
    gk, gv = g.raw_bytes()
    ok, ov = c.valid_bytes()
    assert np.array_equal(host(gk), ok) and np.array_equal(host(gv), ov)
    assert pk.lib().pkv_device_status() == 0, pk.lib().pkv_last_error()
