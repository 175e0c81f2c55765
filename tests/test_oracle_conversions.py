"""Pins the oracle's f16/bf16 conversions (the `half` crate's round-to-nearest-even)
against numpy's IEEE float16 and the bit-level RNE definition of bfloat16."""
import numpy as np


def _interesting_f32():
    rng = np.random.default_rng(0)
    # every f16 value, its neighbours and the midpoints between consecutive f16 values
    h = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16).astype(np.float32)
    f = f[np.isfinite(f)]
    bits = f.view(np.uint32)
    near = np.concatenate([bits, bits + 1, bits - 1]).view(np.float32)
    mids = ((f[:-1].astype(np.float64) + f[1:].astype(np.float64)) / 2).astype(np.float32)
    rand = rng.integers(0, 1 << 32, size=2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65520.0, 65519.99, 6e-8, 3e-8,
                         2.98e-8, 5.96e-8, -5.96e-8, 1e-40, -1e-40], dtype=np.float32)
    out = np.concatenate([near, mids, rand, specials])
    return out[~np.isnan(out)]


def test_f32_to_f16_matches_numpy(orc):
    x = _interesting_f32()
    ours = orc.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    bad = np.nonzero(ours != ref)[0]
    assert bad.size == 0, (x[bad[:5]], ours[bad[:5]], ref[bad[:5]])


def test_f16_to_f32_all_patterns(orc):
    h = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    ours = orc.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(ours[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(ours[np.isnan(ref)]))


def test_f32_to_bf16_round_to_nearest_even(orc):
    x = _interesting_f32()
    u = x.view(np.uint32).astype(np.uint64)
    ref = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)  # RNE on the raw bits
    ours = orc.f32_to_bf16_bits(x)
    assert np.array_equal(ours, ref)
    nan = np.array([np.nan, -np.nan], dtype=np.float32)
    assert np.all((orc.f32_to_bf16_bits(nan) & 0x7FC0) == 0x7FC0)  # stays a quiet NaN


def test_philox_known_answers(orc):
    # Random123 kat_vectors, philox4x32 with 10 rounds
    assert orc.philox([0, 0, 0, 0], [0, 0]) == [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    assert orc.philox([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2) == [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]
    assert orc.philox([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0]) == \
        [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]


def test_normal_generator_closed_form(orc):
    # value = (sum of eight 22-bit draws - 2^24) * sqrt(6) * 2^-23, recomputed from raw Philox
    for seed, stream, idx in [(1, 2, 0), (7, 3, 12345), (2**40 + 5, 2**33 + 1, 2**31 + 3)]:
        c = 2 * idx
        words = []
        for cc in (c, c + 1):
            words += orc.philox([cc & 0xFFFFFFFF, cc >> 32, stream & 0xFFFFFFFF, stream >> 32],
                                [seed & 0xFFFFFFFF, seed >> 32])
        s = sum(w >> 10 for w in words)
        expect = np.float32(s - (1 << 24)) * np.float32(np.sqrt(6.0)) * np.float32(2.0 ** -23)
        got = orc.lib().orc_normal(seed, stream, idx)
        assert np.float32(got) == np.float32(expect)
    x = orc.normal(1 << 20, 11, 5)
    assert abs(x.mean()) < 5e-3 and abs(x.std() - 1) < 5e-3
