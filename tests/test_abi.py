"""libpkv.so loads and exports every entry point that include/pkv.h declares (no GPU
calls: only host-side helpers are exercised)."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "pkv.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pkv_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    from paramecia_amd import _lib
    assert sorted(_lib.SYMBOLS) == header_functions()


def test_library_exports_every_symbol():
    from paramecia_amd import _lib
    L = _lib.lib()
    for name in header_functions():
        assert hasattr(L, name), name
    assert b"gfx950" in L.pkv_version()


def test_host_side_helpers():
    from paramecia_amd import KvCacheQuantization as Q, _lib
    L = _lib.lib()
    for s, q in [("f16", Q.F16), ("FP16", Q.F16), ("bf16", Q.BF16), ("bfloat16", Q.BF16),
                 ("q8", Q.Q8_0), ("Q8_0", Q.Q8_0), ("q4", Q.Q4K), ("q4k", Q.Q4K), ("Q4_K", Q.Q4K),
                 ("none", Q.NONE)]:
        assert Q.from_str(s) == q
    assert Q.from_str("q5") is None
    assert b"q5" in L.pkv_last_error()
    assert Q.default() == Q.Q4K
    assert [Q.F16.block_size(), Q.BF16.block_size(), Q.Q8_0.block_size(), Q.Q4K.block_size()] == [1, 1, 32, 256]
    assert Q.Q4K.to_ggml_dtype() == "Q4K" and Q.F16.to_ggml_dtype() is None
    assert L.pkv_bytes_per_row(4, 256) == 144 and L.pkv_bytes_per_row(3, 256) == 272
    assert L.pkv_bytes_per_row(3, 100) == 4 * 34 and L.pkv_bytes_per_row(1, 256) == 512
    assert L.pkv_quant_is_ggml(4) == 1 and L.pkv_quant_is_ggml(1) == 0


def test_rope_host_tables_match_oracle_bit_exactly(orc):
    """The library's RotaryEmbedding::new restatement (host code, no device work) against
    the oracle's, for the Qwen3-Next shape and an odd theta."""
    import numpy as np
    from paramecia_amd import RotaryEmbedding
    for n_rot, n, theta in [(64, 4096, 1.0e7), (256, 300, 10000.0), (2, 70000, 500000.0)]:
        c, s = RotaryEmbedding.host_tables(n_rot, n, theta)
        oc, os_ = orc.rope_tables(n_rot, n, theta)
        assert np.array_equal(c.numpy().view(np.uint32), oc.view(np.uint32))
        assert np.array_equal(s.numpy().view(np.uint32), os_.view(np.uint32))


def test_rope_host_table_errors():
    import pytest
    from paramecia_amd import KvCacheError, RotaryEmbedding
    with pytest.raises(KvCacheError):
        RotaryEmbedding.host_tables(63, 4, 1e7)
    with pytest.raises(KvCacheError):
        RotaryEmbedding.host_tables(0, 4, 1e7)
