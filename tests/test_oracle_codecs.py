"""Pins the oracle's GGML codecs (restated from candle's k_quants.rs; the candle fork
itself is absent, so byte parity with it stays unpinned) with closed forms, hand-derived
known-answer blocks and format invariants."""
import numpy as np
import pytest

Q8_0, Q4K = 3, 4


def f16(bits):
    return np.array([bits], dtype=np.uint16).view(np.float16).astype(np.float32)[0]


# ---------------------------------------------------------------- Q8_0
def test_q8_0_layout_and_known_answers(orc):
    # amax = 127 -> d = 1 exactly, id = 1: q = f32::round(x), halves away from zero
    x = np.zeros(32, dtype=np.float32)
    x[:12] = [127, -127, 0.5, -0.5, 1.5, 2.5, -2.5, 0.49999997, 3.4999998, -126.5, 63.5, 0.0]
    b = orc.quantize(x, Q8_0)
    assert b.size == 34
    assert b[:2].view(np.uint16)[0] == 0x3C00  # f16(1.0)
    q = b[2:].view(np.int8)
    assert list(q[:12]) == [127, -127, 1, -1, 2, 3, -3, 0, 3, -127, 64, 0]
    assert np.all(q[12:] == 0)


def test_q8_0_zero_block(orc):
    b = orc.quantize(np.zeros(64, dtype=np.float32), Q8_0)
    assert b.size == 68 and np.all(b == 0)


def test_q8_0_closed_form_random(orc):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(32 * 500) * rng.uniform(0.01, 30, 500).repeat(32)).astype(np.float32)
    b = orc.quantize(x, Q8_0).reshape(500, 34)
    xb = x.reshape(500, 32)
    amax = np.abs(xb).max(1)
    d = (amax / np.float32(127)).astype(np.float32)
    assert np.array_equal(b[:, :2].copy().view(np.uint16)[:, 0], d.astype(np.float16).view(np.uint16))
    q = b[:, 2:].view(np.int8).astype(np.int32)
    assert np.abs(q).max() <= 127
    assert np.all(np.abs(q).max(1) == 127)  # the amax element always maps to +-127
    y = orc.dequantize(b.reshape(-1), Q8_0, x.size).reshape(500, 32)
    dq = b[:, :2].copy().view(np.float16).astype(np.float32)
    assert np.array_equal(y, (q * dq).astype(np.float32))  # to_float: q * f32(d)
    # |x - d*q| <= d/2 up to the f16 rounding of d
    err = np.abs(xb - q * d[:, None])
    assert np.all(err <= d[:, None] * 0.5 + 1e-6 * amax[:, None])


def test_q8_0_requantize_idempotent(orc):
    # Q(DQ(b)) == b: amax' = 127*f16(d) so d' = f16(d) and q' = q (reference restore path)
    rng = np.random.default_rng(2)
    x = rng.standard_normal(32 * 4096).astype(np.float32)
    b = orc.quantize(x, Q8_0)
    b2 = orc.quantize(orc.dequantize(b, Q8_0, x.size), Q8_0)
    assert np.array_equal(b, b2)


# ---------------------------------------------------------------- Q4K dequantize
def _pack_scales(ls, lm):
    """GGML Q4K 6-bit scale/min packing, written from the block-format definition."""
    s = np.zeros(12, dtype=np.uint8)
    for j in range(8):
        if j < 4:
            s[j] |= ls[j] & 63
            s[j + 4] |= lm[j] & 63
        else:
            s[j + 4] = (ls[j] & 0xF) | ((lm[j] & 0xF) << 4)
            s[j - 4] |= (ls[j] >> 4) << 6
            s[j] |= (lm[j] >> 4) << 6
    return s


def test_q4k_dequantize_hand_built_block(orc):
    rng = np.random.default_rng(3)
    ls = rng.integers(0, 64, 8)
    lm = rng.integers(0, 64, 8)
    L = rng.integers(0, 16, 256)
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = np.array([0x3C00], dtype=np.uint16).view(np.uint8)   # d = 1.0
    blk[2:4] = np.array([0x3800], dtype=np.uint16).view(np.uint8)   # dmin = 0.5
    blk[4:16] = _pack_scales(ls, lm)
    for c in range(4):
        for l in range(32):
            blk[16 + 32 * c + l] = L[64 * c + l] | (L[64 * c + 32 + l] << 4)
    y = orc.dequantize(blk, Q4K, 256)
    sub = np.arange(256) // 32
    expect = (1.0 * ls[sub]) * L - 0.5 * lm[sub]
    assert np.array_equal(y, expect.astype(np.float32))


# ---------------------------------------------------------------- Q4K quantize
def _header(b):
    return b[0:2].view(np.uint16)[0], b[2:4].view(np.uint16)[0], list(b[4:16])


def test_q4k_known_answer_uniform_block(orc):
    # Every sub-block holds (i % 16) - 8. Hand derivation: make_qkx1_quants returns
    # (scale 1, min 8) after two passes; ls = lm = round(63) = 63; d = f16(1/63) = 0x2410,
    # dmin = f16(8/63) = 0x3010; (x + 7.998046875) / 0.999755859375 rounds to x + 8.
    x = np.tile((np.arange(32) % 16 - 8).astype(np.float32), 8)
    b = orc.quantize(x, Q4K)
    d, dmin, sc = _header(b)
    assert (d, dmin) == (0x2410, 0x3010)
    assert sc == [0xFF] * 12
    qs = b[16:]
    assert list(qs) == [(l % 16) * 0x11 for l in range(32)] * 4


def test_q4k_known_answer_graded_block(orc):
    # Sub-block j holds 2^-(7-j) * ((i % 16) - 8): scale s_j = 2^-(7-j), min 8 s_j (exact).
    # ls = lm = round(63 s_j) = [0, 1, 2, 4, 8, 16, 32, 63] (31.5 -> 32). Sub-block 0 has a
    # zero code, so its nibbles stay 0; the others round back to i % 16.
    base = (np.arange(32) % 16 - 8).astype(np.float32)
    x = np.concatenate([base * np.float32(2.0 ** -(7 - j)) for j in range(8)])
    b = orc.quantize(x, Q4K)
    d, dmin, sc = _header(b)
    assert (d, dmin) == (0x2410, 0x3010)
    assert sc == [0x00, 0x41, 0x82, 0xC4, 0x00, 0x41, 0x82, 0xC4, 0x88, 0x00, 0x00, 0xFF]
    qs = list(b[16:])
    assert qs[:32] == [(l % 16) << 4 for l in range(32)]
    assert qs[32:] == [(l % 16) * 0x11 for l in range(32)] * 3


def test_make_qkx1_quants_exact_grid(orc):
    # x = s*(k - 8) on a power-of-two grid: the fit recovers (s, 8s) exactly
    for e in range(-10, 6):
        s = np.float32(2.0 ** e)
        x = (s * (np.arange(32) % 16 - 8)).astype(np.float32)
        assert orc.make_qkx1_quants(x) == (float(s), float(8 * s))
    # constant sub-block -> (0, 0)
    assert orc.make_qkx1_quants(np.full(32, 3.25, dtype=np.float32)) == (0.0, 0.0)


def _q4k_fields(b):
    b = b.reshape(-1, 144)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dm = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    sc = np.zeros((b.shape[0], 8), dtype=np.int32)
    m = np.zeros_like(sc)
    s = b[:, 4:16].astype(np.int32)
    for j in range(8):
        if j < 4:
            sc[:, j], m[:, j] = s[:, j] & 63, s[:, j + 4] & 63
        else:
            sc[:, j] = (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4)
            m[:, j] = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    return d, dm, sc, m


def test_q4k_invariants_random(orc):
    rng = np.random.default_rng(4)
    n = 2000
    x = rng.standard_normal(256 * n).astype(np.float32)
    x[: 256 * 100] *= 20  # outlier-scale blocks
    b = orc.quantize(x, Q4K)
    assert b.size == 144 * n
    d, dm, sc, m = _q4k_fields(b)
    assert sc.max() <= 63 and m.max() <= 63
    assert np.all(sc.max(1) >= 62)  # the largest sub-block scale maps to ~63
    y = orc.dequantize(b, Q4K, x.size).reshape(n, 8, 32)
    xs = x.reshape(n, 8, 32)
    step = (d[:, None] * sc)[:, :, None]
    err = np.abs(y - xs)
    # each element is within one quantisation step of its sub-block grid
    assert np.all(err <= step * 1.01 + 1e-5 * np.abs(xs).max())
    # N(0,1) sub-blocks: grid step ~ range/15, so the rms error is ~ step/sqrt(12)
    rms = np.sqrt((err[100:] ** 2).mean()) / np.sqrt((xs[100:] ** 2).mean())
    assert rms < 0.1


def test_q4k_constant_subblock_dequantizes_to_zero(orc):
    x = np.random.default_rng(5).standard_normal(256).astype(np.float32)
    x[64:96] = 2.5
    y = orc.dequantize(orc.quantize(x, Q4K), Q4K, 256)
    assert np.all(y[64:96] == 0)


def test_q4k_subblocks_independent_given_header(orc):
    # Permuting the elements inside one sub-block permutes only that sub-block's nibbles
    # when the block-wide maxima do not move.
    rng = np.random.default_rng(6)
    x = rng.standard_normal(256).astype(np.float32)
    b0 = orc.quantize(x, Q4K)
    perm = rng.permutation(32)
    x2 = x.copy()
    x2[96:128] = x[96:128][perm]
    b1 = orc.quantize(x2, Q4K)
    assert np.array_equal(b0[:16], b1[:16])
    y0 = orc.dequantize(b0, Q4K, 256)
    y1 = orc.dequantize(b1, Q4K, 256)
    assert np.array_equal(y0[96:128][perm], y1[96:128])
    assert np.array_equal(np.delete(y0, np.s_[96:128]), np.delete(y1, np.s_[96:128]))


# ---------------------------------------------------------------- Q4K fit, several passes
def _bits(v):
    return int(np.array([v], dtype=np.float32).view(np.uint32)[0])


@pytest.mark.parametrize("name", ["A", "B", "P", "Q"])
def test_make_qkx1_quants_multipass_known_answers(orc, name):
    """Inputs whose fit needs 3 to 5 passes, with rounding ties (A, P), a pass limit that
    decides the result (B, Q) and sums whose order shows in the last bit (A); the per-pass
    derivation is in q4k_known_answers.py."""
    from q4k_known_answers import FITS
    x, scale_bits, neg_min_bits = FITS[name]
    s, m = orc.make_qkx1_quants(np.array(x, dtype=np.float32))
    assert (_bits(s), _bits(m)) == (scale_bits, neg_min_bits)


def test_q4k_block_from_multipass_subblocks(orc):
    from q4k_known_answers import BLOCK_PQ_X, BLOCK_PQ_HEADER, BLOCK_PQ_QS
    b = orc.quantize(np.array(BLOCK_PQ_X, dtype=np.float32), Q4K)
    assert list(b[:16]) == BLOCK_PQ_HEADER
    assert list(b[16:]) == BLOCK_PQ_QS
