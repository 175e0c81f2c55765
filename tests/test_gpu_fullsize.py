"""Full-size GPU parity of the decode and restore paths, with checks that a dropped or
misrouted key range cannot pass (tests/attn_checks.py; shown on the CPU by
test_parity_sensitivity.py):
- one config-3 layer (131072 cached tokens + 1) with a dominant key planted every 128
  keys, so every split range of the decode kernel carries an O(1) share of the output;
- config 5 on one layer at its full seeded lengths (16 sequences, 1024-65536 tokens,
  outlier channels x20), one batched decode step;
- config 4 at full size: 12 full-attention layers of 65536 Q4K tokens and 36 Gated-DeltaNet
  states ([32, 128, 128] ssm, [8192, 3] conv, [32] gate offset) saved, clobbered, restored
  into caches of capacity 131072 and compared byte for byte on the device, then a
  1024-token suffix whose packed rows must equal the oracle's.
Bulk K/V rows are quantized on the GPU and handed to the oracle as bytes (their bit-exact
quantization is tested on its own in test_gpu_decode.py / test_gpu_parity.py); the rows of
every appended token are quantized on both sides and compared."""
import sys

import numpy as np
import pytest

from attn_checks import assert_attn_close, plant, row_errors

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

Q4K = 4


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


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_decode_planted_full_size(pk, orc):
    S = 131072
    say("planted full-size decode: host data")
    rng = np.random.default_rng(31)
    k = rng.standard_normal((1, 2, S, 256), dtype=np.float32)
    v = rng.standard_normal((1, 2, S, 256), dtype=np.float32)
    q = plant(k, v, rng.standard_normal((1, 1, 16, 256), dtype=np.float32), rng)
    kn = rng.standard_normal((1, 2, 1, 256), dtype=np.float32)
    vn = rng.standard_normal((1, 2, 1, 256), dtype=np.float32)
    say("planted full-size decode: GPU quantize + fused step")
    g = pk.PreallocatedQuantizedKvCache(1, 2, S + 1, 256, pk.KvCacheQuantization.Q4K)
    g.append_quantized(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    del k, v
    gk0, gv0 = (host(x) for x in g.raw_bytes())
    out = host(g.append_attend(torch.from_numpy(kn).cuda(), torch.from_numpy(vn).cuda(),
                               torch.from_numpy(q).cuda(), 1 / 16, offset=S))
    gk, gv = (host(x) for x in g.raw_bytes())
    say("planted full-size decode: oracle")
    c = orc.Cache(Q4K, 1, 2, 256, S + 1)
    c.load_bytes(gk0, gv0, S)
    assert c.append(kn, vn) == 0
    ok, ov = c.valid_bytes()
    assert np.array_equal(gk, ok) and np.array_equal(gv, ov), "appended rows differ"
    ref = c.attend(q, 1 / 16, S, True, mode="f64")
    l2, mx = row_errors(out, ref)
    say(f"planted full-size decode: row rel L2 {l2:.2e}, row max {mx:.2e}")
    assert_attn_close(out, ref, what="planted full-size decode")


def test_batched_config5_full_lengths(pk, orc):
    """One layer of config 5 at its real lengths (the decode plan of ~530k keys over 16
    sequences), against the float64 oracle per sequence."""
    from paramecia_amd import workloads as W
    lens = W.c5_lengths()
    chans = W.c5_channels()
    say(f"config 5 full lengths: {sum(lens)} keys over {len(lens)} sequences")
    caches, oracles = [], []
    for i, S in enumerate(lens):
        gc = pk.PreallocatedQuantizedKvCache(1, 2, S + 1, 256, pk.KvCacheQuantization.Q4K)
        kb = torch.empty((1, 2, S, 256), device="cuda")
        vb = torch.empty_like(kb)
        pk.fill_normal(kb, W.SEED, W.stream_id(5, W.T_PREFILL_K, 0, i))
        pk.fill_normal(vb, W.SEED, W.stream_id(5, W.T_PREFILL_V, 0, i))
        pk.scale_channels(kb, chans, W.C5_OUTLIER_SCALE)
        pk.scale_channels(vb, chans, W.C5_OUTLIER_SCALE)
        gc.append_quantized(kb, vb)
        del kb, vb
        c = orc.Cache(Q4K, 1, 2, 256, S + 1)
        c.load_bytes(*(host(x) for x in gc.raw_bytes()), S)
        caches.append(gc)
        oracles.append(c)
    rng = np.random.default_rng(32)
    n = len(lens)
    kn = rng.standard_normal((n, 2, 256), dtype=np.float32)
    vn = rng.standard_normal((n, 2, 256), dtype=np.float32)
    kn[..., chans] *= W.C5_OUTLIER_SCALE
    vn[..., chans] *= W.C5_OUTLIER_SCALE
    q = rng.standard_normal((n, 16, 256), dtype=np.float32)
    say("config 5 full lengths: batched decode step")
    out = host(pk.append_attend_batched(caches, torch.from_numpy(kn).cuda(),
                                        torch.from_numpy(vn).cuda(), torch.from_numpy(q).cuda(),
                                        W.SCALE))
    worst = (0.0, 0.0)
    for i, (gc, c, S) in enumerate(zip(caches, oracles, lens)):
        assert c.append(kn[i][None, :, None], vn[i][None, :, None]) == 0
        ok, ov = c.valid_bytes()
        gk, gv = (host(x) for x in gc.raw_bytes())
        assert np.array_equal(gk, ok) and np.array_equal(gv, ov), f"sequence {i}: rows differ"
        ref = c.attend(q[i][None, None], W.SCALE, S, True, mode="f64")[0, 0]
        e = assert_attn_close(out[i], ref, what=f"config 5 sequence {i} (S={S})")
        worst = (max(worst[0], e[0]), max(worst[1], e[1]))
    say(f"config 5 full lengths: worst row rel L2 {worst[0]:.2e}, row max {worst[1]:.2e}")


def test_prefix_restore_config4_full(pk, orc):
    """Config 4 at full size: the restore of every layer is bit-exact on the device, and the
    1024-token suffix appended after it packs to the oracle's bytes."""
    from paramecia_amd import workloads as W
    S, SUF, cap = 65536, 1024, 131072
    say("config 4 full size: build 12 x 65536 Q4K layers + 36 DeltaNet states")
    m = pk.ModelKvState(W.N_LAYERS, W.FULL_INTERVAL, W.NUM_HEADS, W.NUM_KV_HEADS, W.HEAD_DIM, cap)
    kb = torch.empty((1, 2, S, 256), device="cuda")
    vb = torch.empty_like(kb)
    for i, l in enumerate(m.layers):
        if isinstance(l, pk.FullAttentionKv):
            pk.fill_normal(kb, W.SEED, W.stream_id(4, W.T_PREFILL_K, i))
            pk.fill_normal(vb, W.SEED, W.stream_id(4, W.T_PREFILL_V, i))
            l._ensure(1).append_quantized(kb, vb)
        else:
            ssm = torch.empty((1, W.DN_HEADS, W.DN_DK, W.DN_DV), device="cuda")
            conv = torch.empty((1, W.DN_CONV_DIM, W.DN_CONV_K - 1), device="cuda")
            gate = torch.empty((1, W.DN_HEADS), device="cuda")
            pk.fill_normal(ssm, W.SEED, W.stream_id(4, W.T_SSM, i), 0.02)
            pk.fill_normal(conv, W.SEED, W.stream_id(4, W.T_CONV, i))
            pk.fill_normal(gate, W.SEED, W.stream_id(4, W.T_GATE, i))
            l.recurrent_state = pk.RecurrentState(ssm, conv, gate)
    del kb, vb
    saved = []
    for l in m.layers:
        if isinstance(l, pk.FullAttentionKv):
            saved.append(l.quantized_cache.raw_bytes())
        else:
            rs = l.recurrent_state
            saved.append(tuple(x.clone() for x in (rs.ssm_state, rs.conv_state, rs.gate_cumsum_offset)))
    prefix = m.save_prefix_cache(list(range(S)))
    say("config 4 full size: clobber, then restore into fresh caches of capacity 131072")
    m2 = pk.ModelKvState(W.N_LAYERS, W.FULL_INTERVAL, W.NUM_HEADS, W.NUM_KV_HEADS, W.HEAD_DIM, cap)
    for l in m2.full_layers():  # fresh caches holding other rows, to be overwritten
        l._ensure(1).append_quantized(torch.randn((1, 2, 40, 256), device="cuda"),
                                      torch.randn((1, 2, 40, 256), device="cuda"))
    del m
    assert m2.restore_prefix_cache(prefix) == S
    torch.cuda.synchronize()
    for i, (l, sv) in enumerate(zip(m2.layers, saved)):
        if isinstance(l, pk.FullAttentionKv):
            assert l.cache_seq_len() == S
            rk, rv = l.quantized_cache.raw_bytes()
            assert torch.equal(rk, sv[0]) and torch.equal(rv, sv[1]), f"layer {i}: K/V bytes"
        else:
            rs = l.recurrent_state
            for a, b in zip((rs.ssm_state, rs.conv_state, rs.gate_cumsum_offset), sv):
                assert torch.equal(a, b), f"layer {i}: state"
    say("config 4 full size: 1024-token suffix against the oracle")
    ks = torch.empty((1, 2, SUF, 256), device="cuda")
    vs = torch.empty_like(ks)
    pk.fill_normal(ks, W.SEED, W.stream_id(4, W.T_SUFFIX_K))
    pk.fill_normal(vs, W.SEED, W.stream_id(4, W.T_SUFFIX_V))
    c = orc.Cache(Q4K, 1, 2, 256, SUF)
    assert c.append(host(ks), host(vs)) == 0
    ok, ov = c.valid_bytes()
    row = 2 * 144
    for l in m2.full_layers():
        l.quantized_cache.append_quantized(ks, vs, offset=S)
        gk, gv = (host(x) for x in l.quantized_cache.raw_bytes())
        assert gk.size == (S + SUF) * row
        assert np.array_equal(gk[S * row:], ok) and np.array_equal(gv[S * row:], ov)
