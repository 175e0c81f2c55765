"""GPU parity of the Gated-DeltaNet autoregressive step (pkv_deltanet_step, the role of
delta_net_autoregressive_step, paramecia-model/src/ops.rs:391-403, called at
qwen3_next.rs:3392-3470) against the CPU oracle (orc_deltanet_step) on the same seeded
inputs, through the C ABI and the LinearAttentionState mirror. The reference's kernel is
in the absent candle fork, so parity is tolerance-level: state and output within 1e-4
relative + 2e-6 absolute (state) / 2e-5 absolute (output) of the oracle's f32 result;
the gate offset update is an exact f32 add."""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

RTOL, ATOL_S, ATOL_O = 1e-4, 2e-6, 2e-5
EPS = 1e-6


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


def inputs(rng, b, h, d):
    q = rng.standard_normal((b, h, d)).astype(np.float32)
    k = rng.standard_normal((b, h, d)).astype(np.float32)
    v = rng.standard_normal((b, h, d)).astype(np.float32)
    g = (-np.abs(rng.standard_normal((b, h))) * 0.3).astype(np.float32)
    be = rng.standard_normal((b, h)).astype(np.float32)
    return q, k, v, g, be


def raw_step(pk, q, k, v, g, be, S, go, out, scale):
    from paramecia_amd._lib import lib
    ptr = lambda t: t.data_ptr() if t is not None else None
    return lib().pkv_deltanet_step(ptr(q), ptr(k), ptr(v), ptr(g), ptr(be), ptr(S), ptr(go), ptr(out),
                                   q.shape[0], q.shape[1], q.shape[2], scale, EPS,
                                   torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("b,h,d", [(1, 32, 128), (3, 4, 64), (2, 5, 256), (1, 1, 128)])
def test_step_matches_oracle(pk, orc, b, h, d):
    say(f"deltanet step b={b} h={h} d={d}")
    rng = np.random.default_rng(100 + d + h)
    q, k, v, g, be = inputs(rng, b, h, d)
    S = (rng.standard_normal((b, h, d, d)) * 0.02).astype(np.float32)
    go = rng.standard_normal((b, h)).astype(np.float32)
    scale = d ** -0.5
    Sd, god = dev(S), dev(go)
    out = torch.empty((b, h, d), dtype=torch.float32, device="cuda")
    assert raw_step(pk, dev(q), dev(k), dev(v), dev(g), dev(be), Sd, god, out, scale) == 0
    out_ref = orc.deltanet_step(q, k, v, g, be, S, go, scale, EPS)
    np.testing.assert_allclose(host(out), out_ref, rtol=RTOL, atol=ATOL_O)
    np.testing.assert_allclose(host(Sd), S, rtol=RTOL, atol=ATOL_S)
    np.testing.assert_array_equal(host(god), go)


def test_sequence_through_layer_state(pk, orc):
    """Twelve tokens through LinearAttentionState (zero state on the first, gate offset
    accumulated), the Qwen3-Next shape: 32 value heads x 128, q/k repeated to them."""
    b, h, d = 1, 32, 128
    say("deltanet: 12-token sequence through LinearAttentionState")
    rng = np.random.default_rng(7)
    lin = pk.LinearAttentionState(scale=d ** -0.5, eps=EPS)
    S = np.zeros((b, h, d, d), np.float32)
    go = np.zeros((b, h), np.float32)
    for t in range(12):
        q, k, v, g, be = inputs(rng, b, h, d)
        o = lin.delta_net_autoregressive(dev(q[:, None]), dev(k[:, None]), dev(v[:, None]),
                                         dev(g[:, None]), dev(be[:, None]))
        o_ref = orc.deltanet_step(q, k, v, g, be, S, go, d ** -0.5, EPS)
        assert tuple(o.shape) == (b, 1, h, d)
        np.testing.assert_allclose(host(o)[:, 0], o_ref, rtol=RTOL, atol=ATOL_O)
    rs = lin.recurrent_state
    np.testing.assert_allclose(host(rs.ssm_state), S, rtol=RTOL, atol=ATOL_S)
    np.testing.assert_allclose(host(rs.gate_cumsum_offset), go, rtol=1e-6, atol=1e-6)
    assert tuple(rs.conv_state.shape) == (1, 8192, 3)


def test_edge_cases(pk, orc):
    """beta -> 0 (pure decay), a zero q / k vector (normalised by sqrt(eps)), a strong
    decay, and a null gate offset."""
    b, h, d = 1, 3, 128
    say("deltanet: edge cases")
    rng = np.random.default_rng(8)
    q, k, v, g, be = inputs(rng, b, h, d)
    be[0, 0] = -200.0
    q[0, 1] = 0.0
    k[0, 2] = 0.0
    g[0, 2] = -30.0
    S = (rng.standard_normal((b, h, d, d)) * 0.5).astype(np.float32)
    Sd = dev(S)
    out = torch.empty((b, h, d), dtype=torch.float32, device="cuda")
    assert raw_step(pk, dev(q), dev(k), dev(v), dev(g), dev(be), Sd, None, out, d ** -0.5) == 0
    out_ref = orc.deltanet_step(q, k, v, g, be, S, None, d ** -0.5, EPS)
    np.testing.assert_allclose(host(out), out_ref, rtol=RTOL, atol=ATOL_O)
    np.testing.assert_allclose(host(Sd), S, rtol=RTOL, atol=ATOL_S)


def test_rejects_bad_arguments(pk):
    from paramecia_amd._lib import lib, ERR_ARG, ERR_UNSUPPORTED
    say("deltanet: argument checks")
    b, h = 1, 2
    t = lambda *s: torch.zeros(s, dtype=torch.float32, device="cuda")
    q, k, v, g, be, out = t(b, h, 96), t(b, h, 96), t(b, h, 96), t(b, h), t(b, h), t(b, h, 96)
    S = t(b, h, 96, 96)
    assert raw_step(pk, q, k, v, g, be, S, None, out, 0.1) == ERR_UNSUPPORTED
    assert lib().pkv_deltanet_step(None, k.data_ptr(), v.data_ptr(), g.data_ptr(), be.data_ptr(),
                                   S.data_ptr(), None, out.data_ptr(), b, h, 96, 0.1, EPS,
                                   None) == ERR_ARG
    with pytest.raises(Exception):
        pk.LinearAttentionState().delta_net_autoregressive(t(1, 2, 2, 128), t(1, 2, 2, 128),
                                                           t(1, 2, 2, 128), t(1, 2, 2), t(1, 2, 2))


def test_prefix_snapshot_survives_later_steps(pk):
    """PrefixCache save, two more tokens through every layer (DeltaNet states updated in
    place, K/V appended), restore: the linear layers get the saved states back bit for
    bit (the in-place updates never touched the snapshot), the full layers their saved
    length, and replaying the first post-snapshot token gives the same outputs."""
    say("deltanet: prefix snapshot across in-place steps")
    m = pk.ModelKvState(8, 4, 16, 2, 256, 64)
    lin = [l for l in m.layers if isinstance(l, pk.LinearAttentionState)]
    full = m.full_layers()
    H, D = 32, 128

    def token(seed):
        r = np.random.default_rng(seed)
        kv = [dev(r.standard_normal((1, 2, 1, 256)).astype(np.float32)) for _ in range(2)]
        dn = [tuple(dev(x) for x in (r.standard_normal((1, 1, H, D)).astype(np.float32),
                                     r.standard_normal((1, 1, H, D)).astype(np.float32),
                                     r.standard_normal((1, 1, H, D)).astype(np.float32),
                                     -np.abs(r.standard_normal((1, 1, H))).astype(np.float32),
                                     r.standard_normal((1, 1, H)).astype(np.float32)))
              for _ in lin]
        return kv, dn

    def step(tok):
        kv, dn = tok
        for l in full:
            l._ensure(1).append_quantized(kv[0], kv[1])
        return [host(l.delta_net_autoregressive(*x)) for l, x in zip(lin, dn)]

    for t in range(3):
        step(token(t))
    prefix = m.save_prefix_cache([11, 12, 13])
    saved = [(host(l.recurrent_state.ssm_state), host(l.recurrent_state.gate_cumsum_offset)) for l in lin]
    first = step(token(100))
    step(token(101))
    assert not np.array_equal(host(lin[0].recurrent_state.ssm_state), saved[0][0])
    assert m.restore_prefix_cache(prefix) == 3
    assert m.cache_seq_len() == 3
    for l, (s, g) in zip(lin, saved):
        np.testing.assert_array_equal(host(l.recurrent_state.ssm_state), s)
        np.testing.assert_array_equal(host(l.recurrent_state.gate_cumsum_offset), g)
    again = step(token(100))
    for a, b in zip(first, again):
        np.testing.assert_array_equal(a, b)
