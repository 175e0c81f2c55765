"""Pins the oracle's q/k preparation (RMSNorm + partial RoPE) ahead of the cache.

Reference: FullAttention::forward (paramecia-model/src/qwen3_next.rs:2369-2399):
q_norm / k_norm (candle_nn::ops::rms_norm), then RotaryEmbedding::apply
(qwen3_next.rs:906-940) on the first n_rot = 64 of 256 dims, with the tables of
RotaryEmbedding::new (qwen3_next.rs:878-904). candle itself is absent, so each oracle
function is pinned here by closed forms, special cases, a float64 restatement and the
independent transformers Qwen3-Next implementation (tolerance level).
"""
import numpy as np
import pytest

import oracle as O

THETA = 1.0e7  # Qwen3-Next rope.freq_base
N_ROT, D = 64, 256


# ---------------------------------------------------------------- rope tables
def test_rope_table_position_zero_is_identity():
    c, s = O.rope_tables(N_ROT, 4, THETA)
    assert c.shape == (4, N_ROT // 2)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)


def test_rope_table_closed_form():
    # freq_i = theta^(-2i / n_rot): a base of n_rot / 2 or head_dim, or an exponent of i
    # instead of 2i, is off by far more than the tolerance
    c, s = O.rope_tables(N_ROT, 8, THETA)
    i = np.arange(N_ROT // 2, dtype=np.float64)
    inv = THETA ** (-2.0 * i / N_ROT)
    for t in range(1, 8):
        ang = np.arctan2(s[t].astype(np.float64), c[t].astype(np.float64))
        want = np.angle(np.exp(1j * t * inv))
        assert np.allclose(ang, want, atol=2e-6), t
    assert np.allclose(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2, 1.0, atol=3e-7)


def test_rope_table_matches_transformers():
    torch = pytest.importorskip("torch")
    m = pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
    from transformers import Qwen3NextConfig

    cfg = Qwen3NextConfig(head_dim=D, num_attention_heads=16, num_key_value_heads=2,
                          hidden_size=2048, partial_rotary_factor=0.25, rope_theta=THETA,
                          max_position_embeddings=8192)
    emb = m.Qwen3NextRotaryEmbedding(cfg)
    pos = np.array([0, 1, 2, 17, 1000, 4095, 8191])
    hc, hs = emb(torch.zeros(1, 1, D), torch.tensor(pos)[None])
    c, s = O.rope_tables(N_ROT, 8192, THETA)
    # transformers repeats the 32 frequencies (cat(freqs, freqs)); same f32 product,
    # torch's own cos/sin
    assert np.allclose(hc[0, :, :32].numpy(), c[pos], atol=2e-6)
    assert np.allclose(hc[0, :, 32:].numpy(), c[pos], atol=2e-6)
    assert np.allclose(hs[0, :, :32].numpy(), s[pos], atol=2e-6)


# ---------------------------------------------------------------- rms_norm
def test_rms_norm_constant_and_one_hot_rows():
    eps = 1e-6
    ones = np.ones(D, np.float32)
    x = np.full((1, D), 3.0, np.float32)
    y = O.rms_norm(x, ones, eps)
    assert np.allclose(y, 3.0 / np.sqrt(9.0 + eps), rtol=2e-7)
    # mean, not sum, of squares: [a, 0, ...] -> a / sqrt(a^2 / d + eps)
    x = np.zeros((1, D), np.float32)
    x[0, 0] = 2.0
    y = O.rms_norm(x, ones, eps)
    assert y[0, 0] == pytest.approx(2.0 / np.sqrt(4.0 / D + eps), rel=2e-7)
    assert np.all(y[0, 1:] == 0.0)


def test_rms_norm_sequential_sum_of_squares():
    # 4096^2 = 2^24 comes first; every later 1 is lost to round-to-even in a
    # sequential f32 sum (m = 256 exactly). An exact or pairwise sum gives m =
    # sqrt(65536.996), a reversed order 2^24 + 256.
    eps = 1e-6
    x = np.ones((1, D), np.float32)
    x[0, 0] = 4096.0
    y = O.rms_norm(x, np.ones(D, np.float32), eps)
    assert y[0, 0] == 16.0
    assert np.all(y[0, 1:] == np.float32(1.0 / 256.0))


def test_rms_norm_alpha_per_element_and_float64():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, D)).astype(np.float32) * 2.5
    alpha = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    eps = 1e-6
    y = O.rms_norm(x, alpha, eps)
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd ** 2).mean(-1, keepdims=True) + eps) * alpha
    assert np.allclose(y, want, rtol=1e-6, atol=1e-7)
    # a shifted alpha (a plausible indexing slip) is far off
    assert not np.allclose(y, want / alpha * np.roll(alpha, 1), rtol=1e-3)


def test_rms_norm_matches_transformers():
    torch = pytest.importorskip("torch")
    m = pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
    rng = np.random.default_rng(4)
    w = (0.2 * rng.standard_normal(D)).astype(np.float32)
    norm = m.Qwen3NextRMSNorm(D, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(torch.from_numpy(w))
        x = rng.standard_normal((3, 7, D)).astype(np.float32)
        hf = norm(torch.from_numpy(x)).numpy()
    # GGUF stores the Gemma-style weight with the +1 folded in
    y = O.rms_norm(x, (1.0 + w).astype(np.float32), 1e-6)
    assert np.allclose(y, hf, rtol=3e-6, atol=1e-6)


# ---------------------------------------------------------------- rope
def test_rope_unit_vectors_sign_and_pairing():
    c, s = O.rope_tables(N_ROT, 64, THETA)
    half = N_ROT // 2
    p = 37
    for i in (0, 5, half - 1):
        x = np.zeros((1, D), np.float32)
        x[0, i] = 1.0
        y = O.rope_rows(x, np.array([p]), N_ROT, c, s)
        assert y[0, i] == c[p, i] and y[0, i + half] == s[p, i]
        assert np.count_nonzero(y) == 2
        x = np.zeros((1, D), np.float32)
        x[0, i + half] = 1.0
        y = O.rope_rows(x, np.array([p]), N_ROT, c, s)
        assert y[0, i] == -s[p, i] and y[0, i + half] == c[p, i]


def test_rope_identity_at_zero_and_pass_through():
    c, s = O.rope_tables(N_ROT, 16, THETA)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, D)).astype(np.float32)
    y = O.rope_rows(x, np.zeros(6, np.int64), N_ROT, c, s)
    assert np.array_equal(y, x)
    y = O.rope_rows(x, np.arange(6) + 9, N_ROT, c, s)
    assert np.array_equal(y[:, N_ROT:], x[:, N_ROT:])
    assert not np.array_equal(y[:, :N_ROT], x[:, :N_ROT])


def test_rope_matches_float64_rotation():
    n = 3000
    c, s = O.rope_tables(N_ROT, n, THETA)
    rng = np.random.default_rng(6)
    pos = rng.integers(0, n, size=40)
    x = rng.standard_normal((40, D)).astype(np.float32)
    y = O.rope_rows(x, pos, N_ROT, c, s)
    half = N_ROT // 2
    inv = THETA ** (-2.0 * np.arange(half) / N_ROT)
    z = (x[:, :half] + 1j * x[:, half:N_ROT]).astype(np.complex128)
    z = z * np.exp(1j * pos[:, None].astype(np.float64) * inv)
    # f32 angles p * inv_freq lose ~p * 2^-24 rad
    assert np.allclose(y[:, :half], z.real, atol=5e-4)
    assert np.allclose(y[:, half:N_ROT], z.imag, atol=5e-4)


def test_qk_prep_layout_positions_and_transformers():
    torch = pytest.importorskip("torch")
    m = pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
    rng = np.random.default_rng(7)
    b, l, H, Hkv, off = 2, 5, 16, 2, 11
    q = rng.standard_normal((b, l, H, D)).astype(np.float32)
    k = rng.standard_normal((b, l, Hkv, D)).astype(np.float32)
    qw = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    kw = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    c, s = O.rope_tables(N_ROT, 64, THETA)
    qo, ko = O.qk_prep(q, k, qw, kw, 1e-6, N_ROT, c, s, off)
    # structure: token t of every batch row and head sits at position off + t
    pos_q = np.broadcast_to((off + np.arange(l))[None, :, None], (b, l, H))
    want_q = O.rope_rows(O.rms_norm(q, qw, 1e-6), pos_q.reshape(-1), N_ROT, c, s)
    assert np.array_equal(qo, want_q.reshape(qo.shape))
    pos_k = np.broadcast_to((off + np.arange(l))[None, :, None], (b, l, Hkv))
    want_k = O.rope_rows(O.rms_norm(k, kw, 1e-6), pos_k.reshape(-1), N_ROT, c, s)
    assert np.array_equal(ko, want_k.reshape(ko.shape))
    # transformers: RMSNorm (weight 1 + w) then apply_rotary_pos_emb on [b, h, l, d]
    norm_q = m.Qwen3NextRMSNorm(D, eps=1e-6)
    norm_k = m.Qwen3NextRMSNorm(D, eps=1e-6)
    with torch.no_grad():
        norm_q.weight.copy_(torch.from_numpy(qw - 1.0))
        norm_k.weight.copy_(torch.from_numpy(kw - 1.0))
        tq = norm_q(torch.from_numpy(q)).transpose(1, 2)
        tk = norm_k(torch.from_numpy(k)).transpose(1, 2)
        cc = torch.from_numpy(np.concatenate([c, c], -1)[off:off + l])[None]
        ss = torch.from_numpy(np.concatenate([s, s], -1)[off:off + l])[None]
        hq, hk = m.apply_rotary_pos_emb(tq, tk, cc, ss)
    assert np.allclose(qo, hq.transpose(1, 2).numpy(), rtol=1e-5, atol=2e-6)
    assert np.allclose(ko, hk.transpose(1, 2).numpy(), rtol=1e-5, atol=2e-6)


def test_prep_argument_errors():
    with pytest.raises(ValueError):
        O.rope_tables(63, 4, THETA)
    c, s = O.rope_tables(N_ROT, 4, THETA)
    with pytest.raises(ValueError):
        O.rope_rows(np.zeros((1, 32), np.float32), np.array([0]), N_ROT, c, s)
