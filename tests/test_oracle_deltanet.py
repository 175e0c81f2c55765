"""Pins of the oracle's Gated-DeltaNet step (oracle/pkv_oracle.c: orc_deltanet_step), the
restatement of delta_net_autoregressive_step (paramecia-model/src/ops.rs:391-403) as the
linear-attention layers call it (qwen3_next.rs:3392-3470). The fused CUDA kernel is in the
absent candle fork, so the pins are an independent library routine (transformers'
torch_recurrent_gated_delta_rule, FLA convention: state [dk, dv], beta after sigmoid), a
float64 restatement and closed forms; each catches a transposed state, a dropped decay, a
sign error in the delta or a missing normalisation."""
import numpy as np
import pytest
import torch

import oracle as orc

SCALE = 128 ** -0.5


def inputs(rng, b, h, d, state_std=0.02, gate_std=0.3):
    q = rng.standard_normal((b, h, d)).astype(np.float32)
    k = rng.standard_normal((b, h, d)).astype(np.float32)
    v = rng.standard_normal((b, h, d)).astype(np.float32)
    g = (-np.abs(rng.standard_normal((b, h))) * gate_std).astype(np.float32)
    be = rng.standard_normal((b, h)).astype(np.float32)
    S = (rng.standard_normal((b, h, d, d)) * state_std).astype(np.float32)
    return q, k, v, g, be, S


def step64(q, k, v, g, be, S, scale, eps):
    """float64 restatement, written independently of the C code (state [.., i=v, j=k])."""
    q, k, v, g, be, S = (np.asarray(x, np.float64) for x in (q, k, v, g, be, S))
    qn = q * scale / np.sqrt((q * q).sum(-1, keepdims=True) + eps)
    kn = k / np.sqrt((k * k).sum(-1, keepdims=True) + eps)
    S = S * np.exp(g)[..., None, None]
    u = np.einsum("bhij,bhj->bhi", S, kn)
    d = (v - u) / (1.0 + np.exp(-be))[..., None]
    S = S + d[..., :, None] * kn[..., None, :]
    return np.einsum("bhij,bhj->bhi", S, qn), S


def test_matches_float64_restatement():
    rng = np.random.default_rng(1)
    q, k, v, g, be, S = inputs(rng, 2, 3, 128)
    go = rng.standard_normal((2, 3)).astype(np.float32)
    o64, S64 = step64(q, k, v, g, be, S, SCALE, 1e-6)
    go_ref = go + g
    Sc = S.copy()
    out = orc.deltanet_step(q, k, v, g, be, Sc, go, SCALE, 1e-6)
    np.testing.assert_allclose(out, o64, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(Sc, S64, rtol=1e-5, atol=1e-7)
    np.testing.assert_array_equal(go, go_ref)  # f32 add, same rounding


@pytest.mark.parametrize("steps", [1, 5])
def test_matches_transformers_recurrent_rule(steps):
    from transformers.models.qwen3_next.modeling_qwen3_next import torch_recurrent_gated_delta_rule
    rng = np.random.default_rng(2)
    b, h, d = 2, 4, 128
    S0 = (rng.standard_normal((b, h, d, d)) * 0.02).astype(np.float32)
    qs, ks, vs, gs, bs = [], [], [], [], []
    S = S0.copy()
    go = np.zeros((b, h), np.float32)
    outs = []
    for _ in range(steps):
        q, k, v, g, be, _ = inputs(rng, b, h, d)
        outs.append(orc.deltanet_step(q, k, v, g, be, S, go, SCALE, 1e-6))
        qs.append(q); ks.append(k); vs.append(v); gs.append(g); bs.append(be)
    T = lambda xs: torch.from_numpy(np.stack(xs, 1))  # [b, steps, h, ...]
    o_t, S_t = torch_recurrent_gated_delta_rule(
        T(qs), T(ks), T(vs), T(gs), torch.sigmoid(T(bs)),
        initial_state=torch.from_numpy(S0).transpose(-1, -2).contiguous(),
        output_final_state=True, use_qk_l2norm_in_kernel=True)
    np.testing.assert_allclose(np.stack(outs, 1), o_t.numpy(), rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(S, S_t.transpose(-1, -2).numpy(), rtol=2e-5, atol=2e-7)
    np.testing.assert_allclose(go, np.sum(np.stack(gs, 0), 0), rtol=1e-6, atol=1e-7)


def test_beta_to_zero_is_pure_decay():
    rng = np.random.default_rng(3)
    q, k, v, g, _, S = inputs(rng, 1, 2, 64)
    be = np.full((1, 2), -200.0, np.float32)  # sigmoid underflows to 0 exactly
    Sc = S.copy()
    out = orc.deltanet_step(q, k, v, g, be, Sc, None, SCALE, 1e-6)
    alpha = np.exp(g.astype(np.float64))[..., None, None]
    np.testing.assert_allclose(Sc, S * alpha, rtol=1e-6, atol=0)
    qn = q * SCALE / np.sqrt((q.astype(np.float64) ** 2).sum(-1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(out, np.einsum("bhij,bhj->bhi", S * alpha, qn), rtol=1e-5, atol=1e-7)


def test_zero_state_writes_outer_product():
    rng = np.random.default_rng(4)
    q, k, v, g, be, _ = inputs(rng, 1, 3, 64)
    S = np.zeros((1, 3, 64, 64), np.float32)
    out = orc.deltanet_step(q, k, v, g, be, S, None, SCALE, 1e-6)
    sig = 1.0 / (1.0 + np.exp(-be.astype(np.float64)))
    kn = k / np.sqrt((k.astype(np.float64) ** 2).sum(-1, keepdims=True) + 1e-6)
    qn = q * SCALE / np.sqrt((q.astype(np.float64) ** 2).sum(-1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(S, sig[..., None, None] * v[..., :, None] * kn[..., None, :],
                               rtol=1e-5, atol=1e-8)
    np.testing.assert_allclose(out, sig[..., None] * v * (kn * qn).sum(-1, keepdims=True),
                               rtol=1e-5, atol=1e-7)


def test_one_hot_key_with_full_beta_stores_value():
    """k = e_m, eps = 0, sigmoid(beta) = 1: column m of the decayed state becomes v (the
    delta rule's overwrite), every other column is only decayed."""
    rng = np.random.default_rng(5)
    q, _, v, g, _, S = inputs(rng, 1, 1, 64)
    m = 17
    k = np.zeros((1, 1, 64), np.float32)
    k[0, 0, m] = 3.0  # normalised to exactly 1
    be = np.full((1, 1), 200.0, np.float32)
    Sc = S.copy()
    orc.deltanet_step(q, k, v, g, be, Sc, None, SCALE, 0.0)
    alpha = np.float32(np.exp(np.float32(g[0, 0])))
    np.testing.assert_allclose(Sc[0, 0, :, m], v[0, 0], rtol=0, atol=1e-6)
    others = [j for j in range(64) if j != m]
    np.testing.assert_allclose(Sc[0, 0][:, others], S[0, 0][:, others] * alpha, rtol=1e-6, atol=0)
