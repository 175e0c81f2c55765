"""Pins of the oracle's GGUF weight decoders for the output projection (orc_q5k_dequantize,
orc_q6k_dequantize; the Q4K and Q8_0 decoders are pinned with the cache codecs) and of the
type-generic gated projection orc_gated_oproj (qwen3_next.rs:2657-2680).

The candle fork that decodes these blocks in the reference is absent, and the reference
holds no Q5K/Q6K vectors, so the decoders are pinned against the published block layouts
(ggml-common.h; upstream candle k_quants.rs to_float): blocks packed element by element
by tests/kquant_blocks.py decode to the closed form y = (d * sc) * q - dmin * m (Q5K) or
(d * sc) * (q - 32) (Q6K), every f32 product exact or rounded once, so float64 rounded to
f32 is bit-exact; single-bit perturbations move exactly the element the layout names; a
Q5K block with no high bits decodes as the Q4K block with the same bytes. A swapped nibble,
a high bit or bit pair read for the wrong element, a scale index off by one sub-block, an
unsigned Q6K scale or d read from the wrong end fails one of these."""
import numpy as np
import pytest

import oracle as orc
from kquant_blocks import (W_Q4K, W_Q5K, W_Q6K, W_Q8_0, W_BLOCK_BYTES, pack_q4k, pack_q5k,
                           pack_q6k, pack_q8_0, random_weight_bytes)


def f16(v):
    return np.float64(np.float16(v))


# ---------------------------------------------------------------- Q5K
def test_q5k_hand_built_block_closed_form():
    rng = np.random.default_rng(51)
    for trial in range(6):
        ls, lm = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        codes = rng.integers(0, 32, 256)
        d, dmin = f16(rng.uniform(1e-4, 2.0)), f16(rng.uniform(0, 1.0))
        blk = pack_q5k(d, dmin, ls, lm, codes)
        y = orc.dequantize_weight(blk, W_Q5K, 256)
        sub = np.arange(256) // 32
        # d * sc (17 bits) and (d * sc) * code (22 bits) are exact in f32; the subtraction
        # rounds once, as float64 rounded to f32 does
        expect = ((d * ls[sub]) * codes - dmin * lm[sub]).astype(np.float32)
        assert np.array_equal(y, expect), trial


def test_q5k_high_bit_map():
    # bit j of high-bit byte l adds 16 * d * sc_j to element 32 j + l only
    ls, lm = np.arange(1, 9), np.zeros(8, dtype=np.int64)
    base = pack_q5k(1.0, 0.0, ls, lm, np.zeros(256, dtype=np.int64))
    for l in range(32):
        for j in range(8):
            blk = base.copy()
            blk[16 + l] |= 1 << j
            y = orc.dequantize_weight(blk, W_Q5K, 256)
            nz = np.flatnonzero(y)
            assert list(nz) == [32 * j + l], (l, j, nz)
            assert y[32 * j + l] == 16.0 * ls[j]


def test_q5k_nibble_map():
    ls, lm = np.ones(8, dtype=np.int64), np.zeros(8, dtype=np.int64)
    base = pack_q5k(1.0, 0.0, ls, lm, np.zeros(256, dtype=np.int64))
    for p in range(128):
        for hi in range(2):
            blk = base.copy()
            blk[48 + p] = 1 << (4 * hi)
            y = orc.dequantize_weight(blk, W_Q5K, 256)
            c, l = divmod(p, 32)
            assert list(np.flatnonzero(y)) == [64 * c + 32 * hi + l], (p, hi)


def test_q5k_without_high_bits_is_q4k():
    rng = np.random.default_rng(52)
    for _ in range(4):
        ls, lm = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        codes = rng.integers(0, 16, 256)
        d, dmin = f16(rng.uniform(1e-3, 1.0)), f16(rng.uniform(0, 1.0))
        y5 = orc.dequantize_weight(pack_q5k(d, dmin, ls, lm, codes), W_Q5K, 256)
        y4 = orc.dequantize_weight(pack_q4k(d, dmin, ls, lm, codes), W_Q4K, 256)
        assert np.array_equal(y5, y4)


# ---------------------------------------------------------------- Q6K
def test_q6k_hand_built_block_closed_form():
    rng = np.random.default_rng(61)
    for trial in range(6):
        scales = rng.integers(-128, 128, 16)
        codes = rng.integers(0, 64, 256)
        d = f16(rng.uniform(1e-4, 2.0)) * (1 if trial % 2 else -1)
        blk = pack_q6k(d, scales, codes)
        y = orc.dequantize_weight(blk, W_Q6K, 256)
        # d * sc is exact in f32; the product with (q - 32) rounds once
        expect = ((d * scales[np.arange(256) // 16]) * (codes - 32)).astype(np.float32)
        assert np.array_equal(y, expect), trial


def test_q6k_bit_maps():
    scales = np.ones(16, dtype=np.int64)
    zero = pack_q6k(1.0, scales, np.full(256, 32))  # every value 0
    # the low-nibble array: byte p, nibble hi
    for p in range(128):
        for hi in range(2):
            blk = zero.copy()
            blk[p] ^= 1 << (4 * hi)
            y = orc.dequantize_weight(blk, W_Q6K, 256)
            h, r = divmod(p, 64)
            e = 128 * h + 32 * (r // 32 + 2 * hi) + r % 32
            assert list(np.flatnonzero(y)) == [e], (p, hi)
            assert y[e] == 1.0
    # the high-bit array: byte p, bit pair g
    for p in range(64):
        for g in range(4):
            for bit, val in ((0, 16.0), (1, -32.0)):
                blk = zero.copy()
                blk[128 + p] ^= 1 << (2 * g + bit)
                y = orc.dequantize_weight(blk, W_Q6K, 256)
                h, l = divmod(p, 32)
                e = 128 * h + 32 * g + l
                assert list(np.flatnonzero(y)) == [e], (p, g, bit)
                # code 32 = 0b100000: toggling bit 4 gives 48 (value +16), toggling bit 5
                # gives 0 (value -32)
                assert y[e] == val, (p, g, bit)


def test_q6k_scale_and_d_placement():
    scales = np.arange(-8, 8)  # distinct, signed
    y = orc.dequantize_weight(pack_q6k(0.5, scales, np.full(256, 33)), W_Q6K, 256)
    assert np.array_equal(y, (0.5 * scales[np.arange(256) // 16]).astype(np.float32))
    blk = pack_q6k(1.0, np.ones(16, dtype=np.int64), np.full(256, 33))
    blk[0:2] = 0  # the first bytes are codes, not d: clearing them changes codes 0..3, 64..67
    y = orc.dequantize_weight(blk, W_Q6K, 256)
    assert set(np.flatnonzero(y != 1.0)) == {0, 1, 64, 65}


# ---------------------------------------------------------------- gated projection
ALL = [W_Q8_0, W_Q4K, W_Q5K, W_Q6K]


@pytest.mark.parametrize("w_type", ALL)
def test_gated_oproj_matches_float64(w_type):
    rng = np.random.default_rng(70 + w_type)
    b, in_dim, out_dim = 2, 2048, 24
    wb = random_weight_bytes(rng, w_type, out_dim, in_dim)
    wdq = orc.dequantize_weight(wb, w_type, out_dim * in_dim).reshape(out_dim, in_dim)
    x = rng.standard_normal((b, in_dim)).astype(np.float32)
    g = rng.standard_normal((b, in_dim)).astype(np.float32)
    y64 = (x.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))) @ wdq.astype(np.float64).T
    got = orc.gated_oproj(x, g, wb, w_type, out_dim)
    scale = np.abs(wdq).astype(np.float64) @ np.abs(x[0]).astype(np.float64)
    assert np.all(np.abs(got - y64) <= 1e-5 * scale.max() + 1e-4 * np.abs(y64))
    # the rows: row o of the weights gives output o
    one = orc.gated_oproj(x[:1], None, wb[: wb.size // out_dim * 3], w_type, 3)
    np.testing.assert_allclose(one[0], wdq[:3].astype(np.float64) @ x[0], rtol=1e-4, atol=1e-4)


def test_gated_oproj_q4k_entry_is_generic_q4k():
    rng = np.random.default_rng(80)
    wb = random_weight_bytes(rng, W_Q4K, 8, 4096)
    x = rng.standard_normal((3, 4096)).astype(np.float32)
    g = rng.standard_normal((3, 4096)).astype(np.float32)
    assert np.array_equal(orc.gated_oproj(x, g, wb, W_Q4K, 8), orc.gated_oproj_q4k(x, g, wb, 8))


def test_q8_0_weight_decoder_is_the_cache_decoder():
    codes = np.arange(-16, 16)
    y = orc.dequantize_weight(pack_q8_0(0.25, codes), W_Q8_0, 32)
    assert np.array_equal(y, (0.25 * codes).astype(np.float32))


def test_row_bytes():
    for w_type, per in ((W_Q8_0, 34 * 8), (W_Q4K, 144), (W_Q5K, 176), (W_Q6K, 210)):
        assert orc.lib().orc_weight_row_bytes(w_type, 256) == per
    assert orc.lib().orc_weight_row_bytes(99, 256) == 0
    assert W_BLOCK_BYTES[W_Q6K] == 210
