"""Attention parity checks shared by the tests.

Two gates on every attention output:
- the tolerance the north star states: max-abs 2e-3 / relative 1e-3 against the oracle's
  f32 dequant-then-attend (numpy's assert_allclose form);
- a bound scaled to the output itself, per output row (one query of one head):
  ||got - ref||_2 <= REL_L2 * ||ref||_2 and max|got - ref| <= REL_MAX * max|ref|.

At 131k N(0,1) keys the output's RMS is about 5e-3, so the first gate alone is about 40%
of a typical value and cannot see a missing or doubled range of keys; the second can: a
range of k keys out of S moves a row by about sqrt(k / S) of its norm (512 of 131073
keys: 6%). The kernels' own error against the float64 oracle is about 1e-6 of a row's
norm (operands exact or split into fp16 hi + lo parts, f32 accumulation); REL_L2 and
REL_MAX leave a wide margin above it and stay far below any dropped key range.

planted_layer() builds K/V in which every P-th key dominates the scores and carries a
one-hot V row, so that every range of keys a decode kernel splits off contributes an
O(1) share of the output: a dropped, doubled or misrouted range moves some elements by
a large fraction of their value.
"""
from __future__ import annotations

import numpy as np

ATOL, RTOL = 2e-3, 1e-3
REL_L2 = 2e-5
REL_MAX = 1e-4


def row_errors(got, ref):
    """(worst row relative L2 error, worst row max error / row max |ref|) over the rows of
    the last dimension."""
    g = np.asarray(got, dtype=np.float64).reshape(-1, np.shape(got)[-1])
    r = np.asarray(ref, dtype=np.float64).reshape(-1, np.shape(ref)[-1])
    d = g - r
    rn = np.linalg.norm(r, axis=1)
    l2 = np.linalg.norm(d, axis=1) / np.maximum(rn, 1e-30)
    mx = np.abs(d).max(axis=1) / np.maximum(np.abs(r).max(axis=1), 1e-30)
    return float(l2.max()), float(mx.max())


def assert_attn_close(got, ref, atol=ATOL, rtol=RTOL, rel_l2=REL_L2, rel_max=REL_MAX, what=""):
    np.testing.assert_allclose(np.asarray(got, dtype=np.float64), np.asarray(ref, dtype=np.float64),
                               atol=atol, rtol=rtol, err_msg=what)
    l2, mx = row_errors(got, ref)
    assert l2 <= rel_l2, f"{what}: row relative L2 error {l2:.3e} > {rel_l2:.1e}"
    assert mx <= rel_max, f"{what}: row max error {mx:.3e} of the row's max > {rel_max:.1e}"
    return l2, mx


# ---------------------------------------------------------------- planted keys
PLANT_EVERY = 128      # one dominant key per 128 keys (splits hold 128 keys or more)
PLANT_FIRST = 37       # not aligned with the 32-key blocks
PLANT_V = 8.0          # height of the one-hot V row
PLANT_ALPHA = 1.0      # planted K row = alpha * u_g: score alpha |u_g|^2 / 16 ~ 16 nats


def planted_positions(S: int):
    return np.arange(PLANT_FIRST, S, PLANT_EVERY)


def planted_channel(j: np.ndarray):
    """One-hot channel of planted key number j: a stride that sends neighbouring planted
    keys (and so neighbouring key ranges) to distinct channels."""
    return (np.asarray(j) * 37) % 256


def plant(k: np.ndarray, v: np.ndarray, q: np.ndarray, rng) -> np.ndarray:
    """Plant dominant keys into k, v [B, 2, S, 256] (in place) and return q [B, 1, 16, 256]
    built so that each KV head's 8 query heads share a direction u_g (plus 10% noise):
    planted K rows are alpha * u_g, planted V rows are one-hot PLANT_V at planted_channel."""
    B, H, S, D = k.shape
    pos = planted_positions(S)
    u = rng.standard_normal((B, H, D)).astype(np.float32)
    for b in range(B):
        for g in range(H):
            q[b, 0, 8 * g:8 * g + 8] = u[b, g] + 0.1 * rng.standard_normal((8, D)).astype(np.float32)
            k[b, g, pos] = PLANT_ALPHA * u[b, g]
            v[b, g, pos] = 0.0
            v[b, g, pos, planted_channel(np.arange(pos.size))] = PLANT_V
    return q
