"""The attention checks can fail for the mistakes a split-K decode can make. On the CPU, at
one config-3 layer's size (131073 keys, 16 query heads over 2 KV heads), the exact output
is compared with the output of the same attention with one 512-key range dropped (one
workgroup's share of the decode kernel's split at this size) or counted twice:
- on N(0,1) data the north-star tolerance alone (2e-3 / 1e-3) passes a dropped range,
  while the output-scaled bound of attn_checks rejects it;
- with planted dominant keys (attn_checks.plant) both reject it.
No GPU and no library code: this checks the checks."""
import numpy as np
import pytest

from attn_checks import (ATOL, PLANT_V, RTOL, assert_attn_close, plant, planted_channel,
                         planted_positions)

S = 131073
SPLIT = (65536, 65536 + 512)


def attend(q, k, v, weight=None):
    """float64 softmax(q k^T / 16) v per query head, query head h on KV head h // 8;
    `weight` multiplies each key's softmax term (0 drops a key, 2 counts it twice)."""
    B, _, H, D = q.shape
    out = np.zeros((B, 1, H, D))
    for b in range(B):
        for g in range(k.shape[1]):
            K = k[b, g].astype(np.float64)
            V = v[b, g].astype(np.float64)
            s = np.clip(q[b, 0, 8 * g:8 * g + 8].astype(np.float64) @ K.T / 16.0, -100, 100)
            p = np.exp(s - s.max(axis=1, keepdims=True))
            if weight is not None:
                p = p * weight
            out[b, 0, 8 * g:8 * g + 8] = (p @ V) / p.sum(axis=1, keepdims=True)
    return out


def data(planted):
    rng = np.random.default_rng(11)
    k = rng.standard_normal((1, 2, S, 256), dtype=np.float32)
    v = rng.standard_normal((1, 2, S, 256), dtype=np.float32)
    q = rng.standard_normal((1, 1, 16, 256), dtype=np.float32)
    if planted:
        q = plant(k, v, q, rng)
    return q, k, v


def old_gate_passes(got, ref):
    try:
        np.testing.assert_allclose(got, ref, atol=ATOL, rtol=RTOL)
        return True
    except AssertionError:
        return False


def new_gate_passes(got, ref):
    try:
        assert_attn_close(got, ref)
        return True
    except AssertionError:
        return False


@pytest.fixture(scope="module")
def normal():
    q, k, v = data(False)
    return q, k, v, attend(q, k, v)


@pytest.fixture(scope="module")
def planted():
    q, k, v = data(True)
    return q, k, v, attend(q, k, v)


def weights(factor):
    w = np.ones(S)
    w[SPLIT[0]:SPLIT[1]] = factor
    return w


def test_dropped_split_on_normal_data(normal):
    q, k, v, ref = normal
    got = attend(q, k, v, weights(0.0))
    assert old_gate_passes(got, ref), "the tolerance alone was expected to miss this"
    assert not new_gate_passes(got, ref)
    assert new_gate_passes(ref.astype(np.float32), ref)  # rounding to f32 alone passes


def test_doubled_split_on_normal_data(normal):
    q, k, v, ref = normal
    assert not new_gate_passes(attend(q, k, v, weights(2.0)), ref)


def test_dropped_split_with_planted_keys(planted):
    q, k, v, ref = planted
    got = attend(q, k, v, weights(0.0))
    assert not old_gate_passes(got, ref)
    assert not new_gate_passes(got, ref)
    # planted keys dominate: each channel holds PLANT_V x its share of the planted keys
    pos = planted_positions(S)
    share = np.bincount(planted_channel(np.arange(pos.size)), minlength=256) / pos.size
    np.testing.assert_allclose(ref[0, 0], np.tile(PLANT_V * share, (16, 1)), rtol=1e-4)
