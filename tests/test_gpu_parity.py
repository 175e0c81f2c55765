"""GPU parity tests: libpkv (through its C ABI) against the CPU oracle on the same
seeded inputs. Packed bytes, offsets and restores must be bit-exact; attention must be
within 2e-3 absolute + 1e-3 relative of the oracle's f32 dequant-then-attend."""
import sys

import numpy as np
import pytest

from attn_checks import assert_attn_close

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

F16, BF16, Q8_0, Q4K = 1, 2, 3, 4
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


def special_rows(rng, n_rows, d):
    """Random rows plus the edge cases the codecs must agree on."""
    x = rng.standard_normal((n_rows, d)).astype(np.float32)
    if n_rows >= 12:
        x[0] = 0.0
        x[1, : d // 2] = 3.25                                 # constant sub-blocks
        x[2] = np.round(x[2] * 4) / 4                         # quarter-grid ties
        x[3] *= 1e-30                                         # tiny
        x[4] *= 1e4                                           # huge
        x[5] = np.abs(x[5])                                   # all non-negative
        x[6] = -np.abs(x[6])                                  # all non-positive
        x[7, ::7] *= 20                                       # outlier channels
        x[8] = (np.arange(d) % 16 - 8).astype(np.float32)     # exact grid
        x[9] = np.where(np.arange(d) % 2, 1.0, -1.0)
        x[10, :] = 0.0
        x[10, 5] = 1e-3
        x[11] *= 65504.0 / np.abs(x[11]).max()                # f16 max range
    return x


@pytest.mark.parametrize("quant,B,H,D", [(Q4K, 2, 2, 256), (Q8_0, 2, 2, 256), (F16, 1, 2, 128),
                                         (BF16, 1, 2, 64), (Q8_0, 1, 3, 100), (Q4K, 1, 2, 320)])
def test_append_bytes_and_get_kv_bitexact(pk, orc, quant, B, H, D):
    say(f"append parity quant={quant} B={B} H={H} D={D}")
    rng = np.random.default_rng(100 + quant + D)
    cap = 64
    g = pk.PreallocatedQuantizedKvCache(B, H, cap, D, pk.KvCacheQuantization(quant))
    c = orc.Cache(quant, B, H, D, cap)
    for n in (1, 7, 24):
        k = special_rows(rng, B * H * n, D).reshape(B, H, n, D)
        v = special_rows(rng, B * H * n, D).reshape(B, H, n, D)[:, :, ::-1].copy()
        g.append_quantized(dev(k), dev(v))
        assert c.append(k, v) == 0
    assert g.seq_len == c.seq_len == 32
    gk, gv = g.raw_bytes()
    ok, ov = c.valid_bytes()
    assert np.array_equal(host(gk), ok)
    assert np.array_equal(host(gv), ov)
    k, v = g.get_kv()
    rk, rv = c.get_kv()
    assert np.array_equal(host(k).view(np.uint32), rk.view(np.uint32))
    assert np.array_equal(host(v).view(np.uint32), rv.view(np.uint32))


@pytest.mark.parametrize("quant", [Q4K, Q8_0])
def test_bulk_append_bitexact(pk, orc, quant):
    """Large appends take the throughput kernels, small ones the latency kernels."""
    say(f"bulk append quant={quant}")
    rng = np.random.default_rng(200 + quant)
    g = pk.PreallocatedQuantizedKvCache(1, 2, 2048, 256, pk.KvCacheQuantization(quant))
    c = orc.Cache(quant, 1, 2, 256, 2048)
    for n in (1500, 1, 3):
        k = special_rows(rng, 2 * n, 256).reshape(1, 2, n, 256) * 3
        v = rng.standard_normal((1, 2, n, 256)).astype(np.float32)
        g.append_quantized(dev(k), dev(v))
        assert c.append(k, v) == 0
    gk, gv = g.raw_bytes()
    ok, ov = c.valid_bytes()
    assert np.array_equal(host(gk), ok) and np.array_equal(host(gv), ov)


@pytest.mark.parametrize("D,n", [(256, 300), (320, 150), (256, 1500), (320, 700), (256, 2100),
                                 (320, 1100)])
def test_q4k_append_lane_splits_bitexact(pk, orc, D, n):
    """The throughput kernel at each split of a sub-block's fit over lanes: K and V
    superblocks 1200 (D 256) / 1200 (D 320, two superblocks per row, the second
    zero-padded) run 4 lanes per sub-block, 6000 / 5600 run 2, 8400 / 8800 run 1."""
    say(f"q4k lane-split append D={D} n={n}")
    rng = np.random.default_rng(400 + D + n)
    g = pk.PreallocatedQuantizedKvCache(1, 2, n + 8, D, pk.KvCacheQuantization.Q4K)
    c = orc.Cache(Q4K, 1, 2, D, n + 8)
    k = special_rows(rng, 2 * n, D).reshape(1, 2, n, D) * 3
    v = special_rows(rng, 2 * n, D).reshape(1, 2, n, D)[:, :, ::-1].copy()
    g.append_quantized(dev(k), dev(v))
    assert c.append(k, v) == 0
    gk, gv = g.raw_bytes()
    ok, ov = c.valid_bytes()
    assert np.array_equal(host(gk), ok) and np.array_equal(host(gv), ov)


def nonfinite_rows(rng, n_rows, d):
    """Random rows with NaN and infinities planted: one element, a whole 32-element
    sub-block, every fifth element, both signs."""
    x = rng.standard_normal((n_rows, d)).astype(np.float32)
    plant = [lambda r: r.__setitem__(3, np.nan), lambda r: r.__setitem__(40, np.inf),
             lambda r: r.__setitem__(70, -np.inf), lambda r: r.__setitem__(slice(0, 32), np.nan),
             lambda r: r.__setitem__(slice(None, None, 5), np.inf),
             lambda r: r.__setitem__(0, -np.nan), lambda r: None]
    for i in range(n_rows):
        plant[i % len(plant)](x[i])
    return x


@pytest.mark.parametrize("quant", [Q4K, Q8_0])
def test_append_nonfinite_bitexact(pk, orc, quant):
    """NaN and infinities quantize as the reference's integer conversions fix them (a NaN
    level is 0), through the latency kernels (short appends) and the throughput kernels
    (the 1500-token append)."""
    say(f"non-finite append quant={quant}")
    rng = np.random.default_rng(300 + quant)
    g = pk.PreallocatedQuantizedKvCache(1, 2, 2048, 256, pk.KvCacheQuantization(quant))
    c = orc.Cache(quant, 1, 2, 256, 2048)
    for n in (7, 1500, 2):
        k = nonfinite_rows(rng, 2 * n, 256).reshape(1, 2, n, 256)
        v = nonfinite_rows(rng, 2 * n, 256).reshape(1, 2, n, 256)[:, :, ::-1].copy()
        g.append_quantized(dev(k), dev(v))
        assert c.append(k, v) == 0
    gk, gv = g.raw_bytes()
    ok, ov = c.valid_bytes()
    assert np.array_equal(host(gk), ok) and np.array_equal(host(gv), ov)
    k, v = g.get_kv()
    rk, rv = c.get_kv()
    np.testing.assert_array_equal(host(k), rk)  # NaN matches NaN
    np.testing.assert_array_equal(host(v), rv)


def test_fill_normal_bitexact(pk, orc):
    say("fill_normal parity")
    t = torch.empty(1 << 20, dtype=torch.float32, device="cuda")
    pk.fill_normal(t, 1234, 99, 0.5)
    ref = orc.normal(1 << 20, 1234, 99, 0.5)
    assert np.array_equal(host(t).view(np.uint32), ref.view(np.uint32))


def test_offset_overflow_rules(pk):
    say("offset/overflow rules")
    g = pk.PreallocatedQuantizedKvCache(1, 2, 8, 256, pk.KvCacheQuantization.Q4K)
    kv = lambda n: torch.randn(1, 2, n, 256, device="cuda")
    g.append_quantized(kv(6), kv(6))
    before = [host(x) for x in g.raw_bytes()]
    with pytest.raises(pk.KvCacheOverflow):
        g.append_quantized(kv(3), kv(3))
    assert g.seq_len == 6
    assert all(np.array_equal(a, host(b)) for a, b in zip(before, g.raw_bytes()))
    with pytest.raises(pk.KvCacheOffsetMismatch):
        g.append_quantized(kv(1), kv(1), offset=7)
    g.append_quantized(kv(2), kv(2), offset=4)
    assert g.seq_len == 6
    g.truncate(100)
    assert g.seq_len == 6
    g.clear()
    with pytest.raises(pk.EmptyCacheError):
        g.attend(torch.randn(1, 1, 16, 256, device="cuda"), 1 / 16, 0)
    g.resize_batch(2)
    assert g.batch_size == 2 and g.seq_len == 0


def _attend_case(pk, orc, quant, B, H, Hkv, D, S, L, causal, seed, amp=1.0, fused=False):
    rng = np.random.default_rng(seed)
    g = pk.PreallocatedQuantizedKvCache(B, Hkv, S + L, D, pk.KvCacheQuantization(quant))
    c = orc.Cache(quant, B, Hkv, D, S + L)
    k = (rng.standard_normal((B, Hkv, S, D)) * amp).astype(np.float32)
    v = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    g.append_quantized(dev(k), dev(v))
    assert c.append(k, v) == 0
    q = rng.standard_normal((B, L, H, D)).astype(np.float32)
    scale = float(1 / np.sqrt(D))
    if fused:
        kn = rng.standard_normal((B, Hkv, 1, D)).astype(np.float32)
        vn = rng.standard_normal((B, Hkv, 1, D)).astype(np.float32)
        out = g.append_attend(dev(kn), dev(vn), dev(q), scale)
        assert c.append(kn, vn) == 0
        ref = c.attend(q, scale, S, True, mode="f64")
        gk, _ = g.raw_bytes()
        assert np.array_equal(host(gk), c.valid_bytes()[0])
    else:
        out = g.attend(dev(q), scale, S - L, causal)
        ref = c.attend(q, scale, S - L, causal, mode="f64")
    got = host(out)
    assert_attn_close(got, ref)
    return got, ref


@pytest.mark.parametrize("quant,B,H,Hkv,D,S,L,causal", [
    (Q8_0, 1, 16, 2, 256, 4097, 1, True),    # config 1 shape
    (Q4K, 1, 16, 2, 256, 3000, 1, True),
    (Q4K, 2, 16, 2, 256, 700, 5, True),
    (Q4K, 1, 16, 2, 256, 600, 40, True),     # prefill chunk with q_offset
    (Q8_0, 1, 8, 8, 128, 300, 3, False),
    (F16, 1, 4, 2, 64, 257, 2, True),
    (BF16, 1, 16, 1, 256, 129, 1, True),
    (Q8_0, 1, 2, 1, 512, 90, 1, True),
])
def test_attend_parity(pk, orc, quant, B, H, Hkv, D, S, L, causal):
    say(f"attend parity quant={quant} B={B} H={H}/{Hkv} D={D} S={S} L={L} causal={causal}")
    _attend_case(pk, orc, quant, B, H, Hkv, D, S, L, causal, seed=S + L)


@pytest.mark.parametrize("quant", [Q4K, Q8_0])
def test_append_attend_fused(pk, orc, quant):
    say(f"fused append+attend quant={quant}")
    _attend_case(pk, orc, quant, 1, 16, 2, 256, 5000, 1, True, seed=7, fused=True)


def test_attend_clamp_and_outliers(pk, orc):
    say("attend clamp/outliers")
    _attend_case(pk, orc, Q4K, 1, 16, 2, 256, 1500, 1, True, seed=8, amp=20.0)


def test_flash_attn_stateless_matches_cache(pk):
    say("stateless flash_attn")
    g = pk.PreallocatedQuantizedKvCache(1, 2, 2048, 256, pk.KvCacheQuantization.Q8_0)
    g.append_quantized(torch.randn(1, 2, 2000, 256, device="cuda"),
                       torch.randn(1, 2, 2000, 256, device="cuda"))
    q = torch.randn(1, 3, 16, 256, device="cuda")
    a = g.attend(q, 1 / 16, 1997, True)
    kp, vp, n, st = g.get_kv_storage()
    assert n == 2000 * 2 * 272 and st == (2 * 272, 2 * 272, 272, 1)
    b = pk.flash_attn(pk.KvCacheQuantization.Q8_0, q, kp, vp, st, 1 / 16, 2, 2000, 1997, True)
    assert torch.equal(a, b)


@pytest.mark.parametrize("quant,bpr,L", [(Q8_0, 272, 1), (Q4K, 144, 1), (Q4K, 144, 4),
                                         (Q8_0, 272, 6)])
def test_kv_storage_strides_and_flash_attn_batch2(pk, orc, quant, bpr, L):
    """get_kv_storage at batch 2, where stride_b (one sequence's rows of a token) and
    stride_seq (one token's rows of every sequence) differ: rows addressed through the
    returned strides are the oracle's rows, and flash_attn over those pointers and strides
    matches the oracle's attention (qwen3_next.rs:582-617, ops.rs:756)."""
    say(f"kv_storage + flash_attn batch 2 quant={quant} L={L}")
    B, Hkv, H, D, S = 2, 2, 16, 256, 700
    rng = np.random.default_rng(31 + L)
    g = pk.PreallocatedQuantizedKvCache(B, Hkv, 1024, D, pk.KvCacheQuantization(quant))
    c = orc.Cache(quant, B, Hkv, D, 1024)
    k = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    g.append_quantized(dev(k), dev(v))
    assert c.append(k, v) == 0
    kp, vp, n, st = g.get_kv_storage()
    assert st == (Hkv * bpr, B * Hkv * bpr, bpr, 1) and st[0] != st[1]
    assert n == S * B * Hkv * bpr
    kb, vb = g.raw_bytes()
    hk, hv = host(kb), host(vb)
    ck, cv = c.valid_bytes()
    for t, b, h in [(0, 0, 0), (0, 1, 0), (1, 0, 1), (351, 1, 1), (S - 1, 1, 0), (S - 1, 0, 1)]:
        off = t * st[1] + b * st[0] + h * st[2]
        row = ((t * B + b) * Hkv + h) * bpr  # the reference's seq-major row index
        assert np.array_equal(hk[off:off + bpr], ck[row:row + bpr])
        assert np.array_equal(hv[off:off + bpr], cv[row:row + bpr])
    q = rng.standard_normal((B, L, H, D)).astype(np.float32)
    out = pk.flash_attn(pk.KvCacheQuantization(quant), dev(q), kp, vp, st, 1 / 16, Hkv, S,
                        S - L, True)
    ref = c.attend(q, 1 / 16, S - L, True, mode="f64")
    assert_attn_close(host(out), ref)
    assert torch.equal(out, g.attend(dev(q), 1 / 16, S - L, True))


def test_prefix_restore_bytes_and_requantize(pk, orc):
    say("prefix restore")
    from paramecia_amd import workloads as W
    m = pk.ModelKvState(8, 4, 16, 2, 256, 512, pk.KvCacheQuantization.Q4K)
    rng = np.random.default_rng(9)
    full = m.full_layers()
    for l in full:
        x = rng.standard_normal((2, 1, 2, 300, 256)).astype(np.float32)
        l._ensure(1).append_quantized(dev(x[0]), dev(x[1]))
    states = []
    for l in m.layers:
        if isinstance(l, pk.LinearAttentionState):
            s = pk.RecurrentState(torch.randn(1, 4, 8, 8, device="cuda") * 0.02,
                                  torch.randn(1, 16, 3, device="cuda"), None)
            l.recurrent_state = s
            states.append(s)
    snap = [tuple(host(x) for x in l.quantized_cache.raw_bytes()) for l in full]
    sstate = [(host(s.ssm_state), host(s.conv_state)) for s in states]
    pc = m.save_prefix_cache(list(range(300)))
    assert [e.kind for e in pc.layer_caches].count("FullAttention") == 2
    # diverge, then restore
    for l in full:
        l.quantized_cache.append_quantized(torch.randn(1, 2, 50, 256, device="cuda"),
                                           torch.randn(1, 2, 50, 256, device="cuda"), offset=100)
    m.clear_kv_cache()
    assert m.restore_prefix_cache(pc) == 300
    assert m.cache_seq_len() == 300
    for l, (kb, vb) in zip(full, snap):
        gk, gv = l.quantized_cache.raw_bytes()
        assert np.array_equal(host(gk), kb) and np.array_equal(host(gv), vb)
    lin = [l for l in m.layers if isinstance(l, pk.LinearAttentionState)]
    for l, (ss, cs) in zip(lin, sstate):
        assert np.array_equal(host(l.recurrent_state.ssm_state), ss)
        assert np.array_equal(host(l.recurrent_state.conv_state), cs)
        assert not host(l.recurrent_state.gate_cumsum_offset).any()  # zeros when absent
    # reference semantics: restore = quantize(dequantize(saved))
    assert m.restore_prefix_cache(pc, requantize=True) == 300
    for l, (kb, vb) in zip(full, snap):
        c = orc.Cache(Q4K, 1, 2, 256, 512)
        c.load_bytes(kb, vb, 300)
        k, v = c.get_kv()
        c2 = orc.Cache(Q4K, 1, 2, 256, 512)
        c2.append(k, v)
        gk, gv = l.quantized_cache.raw_bytes()
        assert np.array_equal(host(gk), c2.valid_bytes()[0])
        assert np.array_equal(host(gv), c2.valid_bytes()[1])
    # layer-count mismatch bails before touching anything
    m2 = pk.ModelKvState(4, 4, 16, 2, 256, 512, pk.KvCacheQuantization.Q4K)
    with pytest.raises(pk.PrefixLayerMismatch):
        m2.restore_prefix_cache(pc)


def test_prefix_restore_many_segments(pk):
    """A 64-layer model (16 full, 48 linear layers: 176 copy segments, more than the
    kernel-argument table holds) restores through the device-side segment table; odd
    segment sizes exercise the unaligned tail copy."""
    say("prefix restore, 176 segments")
    m = pk.ModelKvState(64, 4, 16, 2, 256, 256, pk.KvCacheQuantization.Q4K)
    full = m.full_layers()
    for l in full:
        l._ensure(1).append_quantized(torch.randn(1, 2, 37, 256, device="cuda"),
                                      torch.randn(1, 2, 37, 256, device="cuda"))
    states = []
    for l in m.layers:
        if isinstance(l, pk.LinearAttentionState):
            s = pk.RecurrentState(torch.randn(1, 3, 5, 7, device="cuda"),
                                  torch.randn(1, 11, 3, device="cuda"),
                                  torch.randn(1, 3, device="cuda"))
            l.recurrent_state = s
            states.append(tuple(host(x).copy() for x in (s.ssm_state, s.conv_state,
                                                        s.gate_cumsum_offset)))
    snap = [tuple(host(x).copy() for x in l.quantized_cache.raw_bytes()) for l in full]
    pc = m.save_prefix_cache(list(range(37)))
    for l in full:
        l.quantized_cache.append_quantized(torch.randn(1, 2, 5, 256, device="cuda"),
                                           torch.randn(1, 2, 5, 256, device="cuda"), offset=10)
    for l in m.layers:  # diverge the recurrent states in place
        if isinstance(l, pk.LinearAttentionState):
            for x in (l.recurrent_state.ssm_state, l.recurrent_state.conv_state,
                      l.recurrent_state.gate_cumsum_offset):
                x.fill_(5.0)
    m.clear_kv_cache()
    assert m.restore_prefix_cache(pc) == 37
    for l, (kb, vb) in zip(full, snap):
        gk, gv = l.quantized_cache.raw_bytes()
        assert np.array_equal(host(gk), kb) and np.array_equal(host(gv), vb)
    lin = [l for l in m.layers if isinstance(l, pk.LinearAttentionState)]
    for l, (ss, cs, gs) in zip(lin, states):
        st = l.recurrent_state
        assert np.array_equal(host(st.ssm_state), ss)
        assert np.array_equal(host(st.conv_state), cs)
        assert np.array_equal(host(st.gate_cumsum_offset), gs)


def test_prefix_restore_graph_capture(pk):
    """A restore captured into a HIP graph on a stream other than the caches' (as a serving
    loop replays it), with more segments than one kernel-argument table holds: the capture
    completes, and every replay, after eager work has overwritten the caches and states,
    restores them byte for byte."""
    say("prefix restore captured in a graph, 176 segments")
    m = pk.ModelKvState(64, 4, 16, 2, 256, 256, pk.KvCacheQuantization.Q4K)
    full = m.full_layers()
    for l in full:
        l._ensure(1).append_quantized(torch.randn(1, 2, 37, 256, device="cuda"),
                                      torch.randn(1, 2, 37, 256, device="cuda"))
    lin = [l for l in m.layers if isinstance(l, pk.LinearAttentionState)]
    for l in lin:
        l.recurrent_state = pk.RecurrentState(torch.randn(1, 3, 5, 7, device="cuda"),
                                              torch.randn(1, 11, 3, device="cuda"),
                                              torch.randn(1, 3, device="cuda"))
    snap = [tuple(host(x).copy() for x in l.quantized_cache.raw_bytes()) for l in full]
    states = [tuple(host(x).copy() for x in (l.recurrent_state.ssm_state,
                                             l.recurrent_state.conv_state,
                                             l.recurrent_state.gate_cumsum_offset)) for l in lin]
    pc = m.save_prefix_cache(list(range(37)))
    torch.cuda.synchronize()

    def diverge(i):
        for l in full:
            l.quantized_cache.append_quantized(torch.randn(1, 2, 5, 256, device="cuda"),
                                               torch.randn(1, 2, 5, 256, device="cuda"),
                                               offset=10 + i)
        for l in lin:
            for x in (l.recurrent_state.ssm_state, l.recurrent_state.conv_state,
                      l.recurrent_state.gate_cumsum_offset):
                x.fill_(5.0 + i)

    def check(what):
        for l, (kb, vb) in zip(full, snap):
            l.quantized_cache.set_len(37)
            gk, gv = l.quantized_cache.raw_bytes()
            assert np.array_equal(host(gk), kb) and np.array_equal(host(gv), vb), what
        for l, (ss, cs, gs) in zip(lin, states):
            st = l.recurrent_state
            assert np.array_equal(host(st.ssm_state), ss), what
            assert np.array_equal(host(st.conv_state), cs), what
            assert np.array_equal(host(st.gate_cumsum_offset), gs), what

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        assert m.restore_prefix_cache(pc) == 37  # eager, sizes every workspace
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            m.restore_prefix_cache(pc)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for i in range(3):
        diverge(i)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        check(f"replay {i}")


def test_batched_decode_matches_per_sequence(pk, orc):
    say("batched decode")
    rng = np.random.default_rng(10)
    lens = [100, 1500, 37, 800]
    caches, oracles = [], []
    for n in lens:
        g = pk.PreallocatedQuantizedKvCache(1, 2, 2048, 256, pk.KvCacheQuantization.Q4K)
        c = orc.Cache(Q4K, 1, 2, 256, 2048)
        k = rng.standard_normal((1, 2, n, 256)).astype(np.float32)
        v = rng.standard_normal((1, 2, n, 256)).astype(np.float32)
        g.append_quantized(dev(k), dev(v))
        c.append(k, v)
        caches.append(g)
        oracles.append(c)
    kn = rng.standard_normal((4, 2, 256)).astype(np.float32)
    vn = rng.standard_normal((4, 2, 256)).astype(np.float32)
    q = rng.standard_normal((4, 16, 256)).astype(np.float32)
    out = host(pk.append_attend_batched(caches, dev(kn), dev(vn), dev(q), 1 / 16))
    for i, (g, c) in enumerate(zip(caches, oracles)):
        c.append(kn[i][None, :, None], vn[i][None, :, None])
        ref = c.attend(q[i][None, None], 1 / 16, lens[i], True, mode="f64")[0, 0]
        assert_attn_close(out[i], ref)
        assert g.seq_len == lens[i] + 1
        assert np.array_equal(host(g.raw_bytes()[0]), c.valid_bytes()[0])


@pytest.mark.parametrize("quant", [F16, BF16])
def test_float_cache_grows_past_capacity(pk, orc, quant):
    """F16/BF16 caches grow instead of overflowing, as the reference's float cache grows by
    Tensor::cat (qwen3_next.rs:2492-2516): appends past the capacity keep every row
    already stored (bytes equal to an oracle cache with room for all of them), the
    offset rule still rewinds, and attention over the grown cache matches the oracle."""
    say(f"float cache growth quant={quant}")
    rng = np.random.default_rng(31)
    g = pk.PreallocatedQuantizedKvCache(1, 2, 4, 64, pk.KvCacheQuantization(quant))
    c = orc.Cache(quant, 1, 2, 64, 64)
    for n in (3, 5, 1, 20):  # 3 -> 8 -> 9 -> 29 tokens: capacity 4 -> 8 -> 16 -> 32
        k = rng.standard_normal((1, 2, n, 64)).astype(np.float32)
        v = rng.standard_normal((1, 2, n, 64)).astype(np.float32)
        g.append_quantized(dev(k), dev(v))
        assert c.append(k, v) == 0
        assert g.seq_len == c.seq_len and g.max_seq_len >= g.seq_len
    assert g.max_seq_len == 32
    gk, gv = g.raw_bytes()
    rk, rv = c.valid_bytes()
    assert np.array_equal(host(gk), rk) and np.array_equal(host(gv), rv)
    k = rng.standard_normal((1, 2, 2, 64)).astype(np.float32)
    g.append_quantized(dev(k), dev(k), offset=25)  # rewinds to 25, then 27 tokens
    c.truncate(25)
    assert c.append(k, k) == 0 and g.seq_len == 27
    q = rng.standard_normal((1, 1, 8, 64)).astype(np.float32)
    out = host(g.attend(dev(q), 0.125, 26))
    assert_attn_close(out, c.attend(q, 0.125, 26, True, mode="f64"))


def test_allocating_calls_refused_under_capture(pk):
    """Calls that allocate or clear device memory (pkv_create, pkv_resize_batch,
    pkv_prefix_save_full / _linear, pkv_pool_create) return PKV_ERR_UNSUPPORTED on a
    capturing stream, before anything is queued, and work again once the capture ends."""
    say("allocating calls under capture")
    import ctypes
    L = pk.lib()
    g = pk.PreallocatedQuantizedKvCache(1, 2, 64, 256, pk.KvCacheQuantization.Q4K)
    g.append_quantized(torch.randn(1, 2, 8, 256, device="cuda"),
                       torch.randn(1, 2, 8, 256, device="cuda"))
    ssm = torch.zeros(32 * 128 * 128, device="cuda")
    conv = torch.zeros(8192 * 3, device="cuda")
    pre = ctypes.c_void_p()
    assert L.pkv_prefix_create((ctypes.c_uint32 * 1)(7), 1, 2, ctypes.byref(pre)) == 0
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    x = torch.zeros(4, device="cuda")
    torch.cuda.synchronize()
    codes = {}
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            x.add_(1.0)
            s = ctypes.c_void_p(side.cuda_stream)
            h = ctypes.c_void_p()
            codes["create"] = L.pkv_create(4, 1, 2, 256, 64, s, ctypes.byref(h))
            assert not h.value
            g.set_stream(side.cuda_stream)
            codes["resize"] = L.pkv_resize_batch(g.handle, 2)
            codes["save_full"] = L.pkv_prefix_save_full(pre, 0, g.handle)
            codes["save_linear"] = L.pkv_prefix_save_linear(
                pre, 1, ctypes.c_void_p(ssm.data_ptr()), ssm.numel(),
                ctypes.c_void_p(conv.data_ptr()), conv.numel(), None, 32, s)
            p = ctypes.c_void_p()
            codes["pool"] = L.pkv_pool_create(4, 2, 256, 64, 4, s, ctypes.byref(p))
            assert not p.value
    torch.cuda.synchronize()
    assert all(c == 8 for c in codes.values()), codes  # PKV_ERR_UNSUPPORTED
    g.set_stream(torch.cuda.current_stream().cuda_stream)
    assert g.batch_size == 1 and g.seq_len == 8
    assert L.pkv_prefix_entry_kind(pre, 0) == 0 and L.pkv_prefix_entry_kind(pre, 1) == 0
    graph.replay()  # the capture recorded the add only: one replay adds one
    torch.cuda.synchronize()
    assert float(x[0]) == 1.0
    # eager again: every call works
    assert L.pkv_prefix_save_full(pre, 0, g.handle) == 0
    assert L.pkv_prefix_entry_kind(pre, 0) == 1
    assert L.pkv_prefix_free(pre) == 0
    g.resize_batch(2)
    assert g.batch_size == 2
