"""GPU parity of the fused q/k preparation + append (pkv_append_prep, pkv_append_attend_prep)
against the CPU oracle: q_norm / k_norm (candle rms_norm), partial rope at positions
offset + t, then the cache codecs (FullAttention::forward, qwen3_next.rs:2369-2442).
Prepared q, cache bytes and rope tables must be bit-exact; attention within 2e-3 absolute
+ 1e-3 relative of the oracle's f32 dequant-then-attend."""
import ctypes
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

F16, BF16, Q8_0, Q4K = 1, 2, 3, 4
ATOL, RTOL = 2e-3, 1e-3
THETA, EPS = 1.0e7, 1e-6


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


def rows(rng, shape):
    """Projection-like rows with the edge cases the norm and codecs must agree on."""
    x = rng.standard_normal(shape).astype(np.float32)
    flat = x.reshape(-1, shape[-1])
    if flat.shape[0] >= 8:
        flat[0] = 0.0                      # m = sqrt(eps)
        flat[1] *= 1e-30                   # squares underflow
        flat[2] *= 1e4
        flat[3, ::5] *= 30.0               # outlier channels
        flat[4] = 2.0                      # constant row
        flat[5] = np.round(flat[5] * 4) / 4
    return x


class Layer:
    """Per-layer weights and the oracle's view of the same preparation."""

    def __init__(self, pk, orc, D, n_rot, max_pos, seed):
        rng = np.random.default_rng(seed)
        self.qa = (1.0 + 0.2 * rng.standard_normal(D)).astype(np.float32)
        self.ka = (1.0 + 0.2 * rng.standard_normal(D)).astype(np.float32)
        self.rope = pk.RotaryEmbedding(n_rot, max_pos, THETA)
        self.prep = pk.QkPrep(dev(self.qa), dev(self.ka), EPS, self.rope)
        self.cos, self.sin = orc.rope_tables(n_rot, max_pos, THETA)
        self.n_rot = n_rot

    def oracle(self, orc, q, k, offset):
        return orc.qk_prep(q, k, self.qa, self.ka, EPS, self.n_rot, self.cos, self.sin, offset)


def oracle_append(c, kp, v):
    """The oracle cache takes [b, h, n, d]: the reference's transposes."""
    assert c.append(np.ascontiguousarray(kp.transpose(0, 2, 1, 3)),
                    np.ascontiguousarray(v.transpose(0, 2, 1, 3))) == 0


def same_bytes(g, c):
    gk, gv = g.raw_bytes()
    ok, ov = c.valid_bytes()
    assert np.array_equal(host(gk), ok)
    assert np.array_equal(host(gv), ov)


def test_rope_device_tables_bitexact(pk, orc):
    say("rope device tables")
    r = pk.RotaryEmbedding(64, 5000, THETA)
    c, s = r.tables()
    oc, os_ = orc.rope_tables(64, 5000, THETA)
    assert np.array_equal(host(c).view(np.uint32), oc.view(np.uint32))
    assert np.array_equal(host(s).view(np.uint32), os_.view(np.uint32))


@pytest.mark.parametrize("quant,B,Hkv,D,n_rot", [
    (Q4K, 2, 2, 256, 64), (Q8_0, 1, 2, 256, 64), (F16, 1, 2, 128, 32), (BF16, 1, 2, 128, 128),
    (Q8_0, 1, 3, 100, 20), (Q4K, 1, 2, 320, 64), (Q4K, 1, 1, 256, 256)])
def test_prep_append_bitexact(pk, orc, quant, B, Hkv, D, n_rot):
    say(f"prep append quant={quant} B={B} Hkv={Hkv} D={D} n_rot={n_rot}")
    rng = np.random.default_rng(300 + quant + D + n_rot)
    H = 4 * Hkv
    cap = 96
    L = Layer(pk, orc, D, n_rot, 128, 7 + quant)
    g = pk.PreallocatedQuantizedKvCache(B, Hkv, cap, D, pk.KvCacheQuantization(quant))
    c = orc.Cache(quant, B, Hkv, D, cap)
    for n, off in [(1, -1), (7, -1), (24, -1), (9, 20), (3, -1)]:
        q = rows(rng, (B, n, H, D))
        k = rows(rng, (B, n, Hkv, D))
        v = rows(rng, (B, n, Hkv, D))
        pos0 = c.seq_len if off < 0 else off
        if off >= 0:
            c.truncate(off)
        qp_ref, kp_ref = L.oracle(orc, q, k, pos0)
        qp = g.append_prep(dev(q), dev(k), dev(v), L.prep, off)
        oracle_append(c, kp_ref, v)
        assert g.seq_len == c.seq_len
        assert np.array_equal(host(qp).view(np.uint32), qp_ref.view(np.uint32))
    same_bytes(g, c)


@pytest.mark.parametrize("quant,B,n_rot", [(Q4K, 1, 64), (Q4K, 2, 64), (Q4K, 5, 64), (Q4K, 1, 128),
                                           (Q4K, 1, 256), (Q8_0, 1, 64),
                                           (F16, 1, 64)])
def test_append_attend_prep_decode(pk, orc, quant, B, n_rot):
    """Prefill from projections (l = 300), then decode steps; every step's output against
    the oracle's attention over its own cache. Q4K with n_rot <= 128 runs the preparation
    inside the decode kernel, the rest through the prep-append kernel."""
    say(f"prep decode quant={quant} B={B} n_rot={n_rot}")
    rng = np.random.default_rng(400 + quant + B + n_rot)
    Hkv, H, D = 2, 16, 256
    L = Layer(pk, orc, D, n_rot, 1024, 11)
    g = pk.PreallocatedQuantizedKvCache(B, Hkv, 512, D, pk.KvCacheQuantization(quant))
    c = orc.Cache(quant, B, Hkv, D, 512)
    q = rows(rng, (B, 300, H, D))
    k = rows(rng, (B, 300, Hkv, D))
    v = rows(rng, (B, 300, Hkv, D))
    _, kp = L.oracle(orc, q, k, 0)
    g.append_prep(None, dev(k), dev(v), L.prep)
    oracle_append(c, kp, v)
    for step in range(3):
        q = rows(rng, (B, 1, H, D))
        k = rows(rng, (B, 1, Hkv, D))
        v = rows(rng, (B, 1, Hkv, D))
        qp, kp = L.oracle(orc, q, k, c.seq_len)
        out = g.append_attend_prep(dev(q), dev(k), dev(v), L.prep, 1.0 / 16.0)
        oracle_append(c, kp, v)
        ref = c.attend(qp, 1.0 / 16.0, c.seq_len - 1, causal=True)
        got = host(out)
        assert np.allclose(got, ref, atol=ATOL, rtol=RTOL), (step, np.abs(got - ref).max())
    same_bytes(g, c)


def test_forward_projected_chunk_then_decode(pk, orc):
    """FullAttentionKv from the projection outputs: a 40-token chunk (causal over the
    chunk) after a 100-token prefix, then one decode step."""
    say("forward_projected")
    rng = np.random.default_rng(500)
    B, Hkv, H, D = 1, 2, 16, 256
    L = Layer(pk, orc, D, 64, 1024, 13)
    fa = pk.FullAttentionKv(H, Hkv, D, 512, pk.KvCacheQuantization.Q4K)
    c = orc.Cache(Q4K, B, Hkv, D, 512)
    pos = 0
    for l in (100, 40, 1):
        q = rows(rng, (B, l, H, D))
        k = rows(rng, (B, l, Hkv, D))
        v = rows(rng, (B, l, Hkv, D))
        qp, kp = L.oracle(orc, q, k, pos)
        out = fa.forward_projected(dev(q), dev(k), dev(v), pos, L.prep)
        oracle_append(c, kp, v)
        ref = c.attend(qp, 1.0 / 16.0, c.seq_len - l, causal=True).reshape(B, l, H * D)
        got = host(out)
        assert np.allclose(got, ref, atol=ATOL, rtol=RTOL), (l, np.abs(got - ref).max())
        pos += l
    assert fa.cache_seq_len() == 141


def test_prep_errors_leave_cache_unchanged(pk, orc):
    say("prep errors")
    rng = np.random.default_rng(600)
    L = Layer(pk, orc, 256, 64, 16, 17)
    g = pk.PreallocatedQuantizedKvCache(1, 2, 64, 256, pk.KvCacheQuantization.Q4K)
    k = rows(rng, (1, 10, 2, 256))
    g.append_prep(None, dev(k), dev(k), L.prep)
    before = [host(t) for t in g.raw_bytes()]
    # positions 10..20 run past the 16-entry rope table
    with pytest.raises(pk.KvCacheError):
        g.append_prep(None, dev(k), dev(k), L.prep)
    assert g.seq_len == 10
    # offset mismatch (offset > len)
    with pytest.raises(pk.KvCacheOffsetMismatch):
        g.append_prep(None, dev(k[:, :1]), dev(k[:, :1]), L.prep, offset=12)
    assert g.seq_len == 10
    after = [host(t) for t in g.raw_bytes()]
    assert all(np.array_equal(a, b) for a, b in zip(before, after))
    # n_rot wider than head_dim
    wide = pk.QkPrep(dev(np.ones(64, np.float32)), dev(np.ones(64, np.float32)), EPS,
                     pk.RotaryEmbedding(128, 16, THETA))
    g2 = pk.PreallocatedQuantizedKvCache(1, 2, 8, 64, pk.KvCacheQuantization.F16)
    with pytest.raises(pk.KvCacheError):
        g2.append_prep(None, dev(k[:, :1, :, :64]), dev(k[:, :1, :, :64]), wide)
    # q without q_out (C ABI)
    from paramecia_amd import _lib
    qd = dev(rows(rng, (1, 1, 8, 256)))
    kd = dev(k[:, :1])
    rc = _lib.lib().pkv_append_prep(g.handle, ctypes.byref(L.prep.c), ctypes.c_void_p(qd.data_ptr()),
                                    8, None, ctypes.c_void_p(kd.data_ptr()),
                                    ctypes.c_void_p(kd.data_ptr()), 1, -1)
    assert rc == _lib.ERR_ARG
    assert g.seq_len == 10
