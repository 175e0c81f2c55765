"""Pins the oracle's cache layout and error rules against their closed forms
(qwen3_next.rs:384-509, 620-642, 2430-2440)."""
import numpy as np
import pytest

F16, BF16, Q8_0, Q4K = 1, 2, 3, 4


@pytest.mark.parametrize("quant,head_dim", [(Q4K, 256), (Q8_0, 256), (F16, 64), (BF16, 128),
                                            (Q8_0, 100), (Q4K, 320)])
def test_row_layout_closed_form(orc, quant, head_dim):
    B, H, n = 2, 3, 5
    rng = np.random.default_rng(10)
    c = orc.Cache(quant, B, H, head_dim, 16)
    bpr = c.bytes_per_row
    block = {Q4K: 256, Q8_0: 32, F16: 1, BF16: 1}[quant]
    padded = -(-head_dim // block) * block
    assert bpr == orc.bytes_per_row(quant, head_dim)
    assert bpr == {Q4K: padded // 256 * 144, Q8_0: padded // 32 * 34, F16: 2 * padded,
                   BF16: 2 * padded}[quant]
    k0 = rng.standard_normal((B, H, 3, head_dim)).astype(np.float32)
    v0 = rng.standard_normal((B, H, 3, head_dim)).astype(np.float32)
    assert c.append(k0, v0) == 0
    k1 = rng.standard_normal((B, H, n, head_dim)).astype(np.float32)
    v1 = rng.standard_normal((B, H, n, head_dim)).astype(np.float32)
    assert c.append(k1, v1) == 0
    assert c.seq_len == 3 + n
    kb, vb = c.valid_bytes()
    assert kb.size == (3 + n) * B * H * bpr
    for t in range(3 + n):
        for b in range(B):
            for h in range(H):
                r = (t * B + b) * H + h  # seq-major row index (qwen3_next.rs:496-498)
                src_k = (k0 if t < 3 else k1)[b, h, t if t < 3 else t - 3]
                src_v = (v0 if t < 3 else v1)[b, h, t if t < 3 else t - 3]
                pad = np.zeros(padded, dtype=np.float32)
                pad[:head_dim] = src_k
                assert np.array_equal(kb[r * bpr:(r + 1) * bpr], orc.quantize(pad, quant))
                pad[:head_dim] = src_v
                assert np.array_equal(vb[r * bpr:(r + 1) * bpr], orc.quantize(pad, quant))
    k, v = c.get_kv()
    assert k.shape == (B, H, 3 + n, head_dim)
    row = kb[((4 * B + 1) * H + 2) * bpr:][:bpr]
    assert np.array_equal(k[1, 2, 4], orc.dequantize(row, quant, padded)[:head_dim])


def test_overflow_and_offset_rules(orc):
    c = orc.Cache(Q4K, 1, 2, 256, 8)
    rng = np.random.default_rng(11)
    kv = lambda n: rng.standard_normal((1, 2, n, 256)).astype(np.float32)
    assert c.append(kv(6), kv(6)) == 0
    before = c.valid_bytes()
    assert c.append(kv(3), kv(3)) == orc.ERR_OVERFLOW  # 9 > 8: no partial write
    assert c.seq_len == 6
    assert all(np.array_equal(a, b) for a, b in zip(before, c.valid_bytes()))
    assert c.append_at(kv(1), kv(1), 7) == orc.ERR_OFFSET  # offset beyond length
    assert c.append_at(kv(2), kv(2), 4) == 0  # smaller offset truncates first
    assert c.seq_len == 6
    c.truncate(10)
    assert c.seq_len == 6  # truncate never grows
    c.truncate(2)
    assert c.seq_len == 2
    c.clear()
    assert c.seq_len == 0
    assert c.resize_batch(3) == 0 and c.seq_len == 0
