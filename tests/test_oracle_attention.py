"""Pins the oracle's attention against an independent numpy softmax(QK^T)V."""
import numpy as np
import pytest

Q8_0, Q4K = 3, 4


def numpy_sdpa(K, V, q, scale, q_offset, causal):
    B, Hkv, S, D = K.shape
    _, L, H, _ = q.shape
    G = H // Hkv
    out = np.zeros(q.shape, dtype=np.float64)
    for b in range(B):
        for h in range(H):
            s = q[b, :, h].astype(np.float64) @ K[b, h // G].astype(np.float64).T * scale
            if causal:
                j = np.arange(S)[None, :]
                i = np.arange(L)[:, None]
                s = np.where(j <= i + q_offset, s, -np.inf)
            s = np.clip(s, -100, 100)
            p = np.exp(s - s.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            out[b, :, h] = p @ V[b, h // G].astype(np.float64)
    return out


@pytest.mark.parametrize("quant,B,H,Hkv,D,S,L,causal,amp", [
    (Q4K, 1, 16, 2, 256, 97, 1, True, 1.0),
    (Q8_0, 2, 8, 2, 64, 50, 4, True, 1.0),
    (Q8_0, 1, 4, 4, 128, 33, 3, False, 1.0),
    (Q4K, 1, 16, 2, 256, 40, 6, True, 30.0),   # large scores hit the +-100 clamp
])
def test_attention_matches_numpy(orc, quant, B, H, Hkv, D, S, L, causal, amp):
    rng = np.random.default_rng(12)
    c = orc.Cache(quant, B, Hkv, D, S)
    k = (rng.standard_normal((B, Hkv, S, D)) * amp).astype(np.float32)
    v = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    assert c.append(k, v) == 0
    q = (rng.standard_normal((B, L, H, D)) * amp).astype(np.float32)
    K, V = c.get_kv()
    q_offset = S - L
    scale = 1.0 / np.sqrt(D)
    ref = numpy_sdpa(K, V, q, scale, q_offset, causal)
    o64 = c.attend(q, scale, q_offset, causal, mode="f64")
    np.testing.assert_allclose(o64, ref, rtol=1e-9, atol=1e-9)
    o32 = c.attend(q, scale, q_offset, causal, mode="f32")
    np.testing.assert_allclose(o32, ref, rtol=1e-4, atol=1e-5)
    ofa = c.attend(q, scale, q_offset, causal, mode="faithful", threads=2)
    np.testing.assert_allclose(ofa, ref, rtol=1e-4, atol=1e-5)
