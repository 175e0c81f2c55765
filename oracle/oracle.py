"""ctypes front end of the CPU oracle (oracle/pkv_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, always as the checker. The product (paramecia_amd) never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpkv_oracle.so")

F16, BF16, Q8_0, Q4K = 1, 2, 3, 4
OK, ERR_OVERFLOW, ERR_OFFSET, ERR_ARG = 0, 1, 2, 3

_lib = None


def build() -> None:
    subprocess.check_call(["make", "-s", "-C", HERE])


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


class OrcCache(ctypes.Structure):
    _fields_ = [
        ("quant", ctypes.c_int),
        ("batch", ctypes.c_int),
        ("n_kv_heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("padded_head_dim", ctypes.c_int),
        ("block", ctypes.c_int),
        ("max_seq_len", ctypes.c_int64),
        ("seq_len", ctypes.c_int64),
        ("bytes_per_row", ctypes.c_size_t),
        ("k", ctypes.POINTER(ctypes.c_uint8)),
        ("v", ctypes.POINTER(ctypes.c_uint8)),
    ]


_fp = ctypes.POINTER(ctypes.c_float)
_dp = ctypes.POINTER(ctypes.c_double)
_u8p = ctypes.POINTER(ctypes.c_uint8)


def _declare(L: ctypes.CDLL) -> None:
    sz, i64, u64 = ctypes.c_size_t, ctypes.c_int64, ctypes.c_uint64
    L.orc_f32_to_f16.argtypes, L.orc_f32_to_f16.restype = [ctypes.c_float], ctypes.c_uint16
    L.orc_f16_to_f32.argtypes, L.orc_f16_to_f32.restype = [ctypes.c_uint16], ctypes.c_float
    L.orc_f32_to_bf16.argtypes, L.orc_f32_to_bf16.restype = [ctypes.c_float], ctypes.c_uint16
    L.orc_bf16_to_f32.argtypes, L.orc_bf16_to_f32.restype = [ctypes.c_uint16], ctypes.c_float
    _u16p = ctypes.POINTER(ctypes.c_uint16)
    for name in ("orc_f32_to_f16_n", "orc_f32_to_bf16_n"):
        getattr(L, name).argtypes = [_fp, _u16p, sz]
    L.orc_f16_to_f32_n.argtypes = [_u16p, _fp, sz]
    for name in ("orc_q8_0_quantize", "orc_q4k_quantize"):
        getattr(L, name).argtypes = [_fp, _u8p, sz]
    for name in ("orc_q8_0_dequantize", "orc_q4k_dequantize", "orc_q5k_dequantize",
                 "orc_q6k_dequantize"):
        getattr(L, name).argtypes = [_u8p, _fp, sz]
    L.orc_make_qkx1_quants.argtypes = [_fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _fp, _fp]
    L.orc_philox4x32_10.argtypes = [ctypes.POINTER(ctypes.c_uint32)] * 3
    L.orc_normal.argtypes, L.orc_normal.restype = [u64, u64, u64], ctypes.c_float
    L.orc_fill_normal.argtypes = [_fp, sz, u64, u64, ctypes.c_float]
    L.orc_bytes_per_row.argtypes, L.orc_bytes_per_row.restype = [ctypes.c_int, ctypes.c_int], sz
    cp = ctypes.POINTER(OrcCache)
    L.orc_cache_init.argtypes = [cp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, i64]
    L.orc_cache_free.argtypes = [cp]
    L.orc_cache_append.argtypes = [cp, _fp, _fp, i64]
    L.orc_cache_append_at.argtypes = [cp, _fp, _fp, i64, i64]
    L.orc_cache_truncate.argtypes = [cp, i64]
    L.orc_cache_clear.argtypes = [cp]
    L.orc_cache_resize_batch.argtypes = [cp, ctypes.c_int]
    L.orc_cache_get_kv.argtypes = [cp, _fp, _fp]
    L.orc_attend_f32.argtypes = [cp, _fp, ctypes.c_int, ctypes.c_int, ctypes.c_float, i64,
                                 ctypes.c_int, _fp, ctypes.c_int]
    L.orc_attend_f64.argtypes = [cp, _fp, ctypes.c_int, ctypes.c_int, ctypes.c_double, i64,
                                 ctypes.c_int, _dp]
    L.orc_attend_faithful.argtypes = [cp, _fp, ctypes.c_int, ctypes.c_int, ctypes.c_float, i64,
                                      ctypes.c_int, _fp, ctypes.c_int]
    _i64p = ctypes.POINTER(ctypes.c_int64)
    L.orc_rope_tables.argtypes = [ctypes.c_int, i64, ctypes.c_double, _fp, _fp]
    L.orc_rms_norm.argtypes = [_fp, _fp, ctypes.c_float, sz, ctypes.c_int, _fp]
    L.orc_rms_norm.restype = None
    L.orc_rope_rows.argtypes = [_fp, sz, ctypes.c_int, ctypes.c_int, _i64p, _fp, _fp]
    L.orc_deltanet_step.argtypes = [_fp] * 8 + [ctypes.c_int] * 3 + [ctypes.c_float] * 2
    L.orc_gated_oproj_q4k.argtypes = [_fp, _fp, _u8p, _fp] + [ctypes.c_int] * 3
    L.orc_gated_oproj.argtypes = [_fp, _fp, _u8p, ctypes.c_int, _fp] + [ctypes.c_int] * 3
    L.orc_weight_row_bytes.argtypes = [ctypes.c_int, ctypes.c_int]
    L.orc_weight_row_bytes.restype = sz
    L.orc_qk_prep.argtypes = [_fp, _fp] + [ctypes.c_int] * 5 + [_fp, _fp, ctypes.c_float,
                                                                 ctypes.c_int, _fp, _fp, i64,
                                                                 _fp, _fp]


def _f(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_fp)


def _u8(a: np.ndarray):
    assert a.dtype == np.uint8 and a.flags.c_contiguous
    return a.ctypes.data_as(_u8p)


# ---------------------------------------------------------------- codecs
BLOCK = {Q8_0: 32, Q4K: 256, F16: 1, BF16: 1}
BLOCK_BYTES = {Q8_0: 34, Q4K: 144}


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(x.size, dtype=np.uint16)
    lib().orc_f32_to_f16_n(_f(x), out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), x.size)
    return out


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(x.size, dtype=np.uint16)
    lib().orc_f32_to_bf16_n(_f(x), out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16).reshape(-1)
    out = np.empty(h.size, dtype=np.float32)
    lib().orc_f16_to_f32_n(h.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), _f(out), h.size)
    return out


def quantize(x: np.ndarray, quant: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    n = x.size
    if quant in (F16, BF16):
        bits = f32_to_f16_bits(x) if quant == F16 else f32_to_bf16_bits(x)
        return bits.view(np.uint8)
    out = np.zeros(n // BLOCK[quant] * BLOCK_BYTES[quant], dtype=np.uint8)
    fn = lib().orc_q8_0_quantize if quant == Q8_0 else lib().orc_q4k_quantize
    fn(_f(x), _u8(out), n)
    return out


def dequantize(b: np.ndarray, quant: int, n: int) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint8)
    if quant == F16:
        return b.view(np.uint16).view(np.float16).astype(np.float32)
    if quant == BF16:
        return (b.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    y = np.zeros(n, dtype=np.float32)
    fn = lib().orc_q8_0_dequantize if quant == Q8_0 else lib().orc_q4k_dequantize
    fn(_u8(b), _f(y), n)
    return y


def make_qkx1_quants(x: np.ndarray, nmax: int = 15, ntry: int = 5):
    x = np.ascontiguousarray(x, dtype=np.float32)
    s, m = ctypes.c_float(), ctypes.c_float()
    lib().orc_make_qkx1_quants(_f(x), x.size, nmax, ntry, ctypes.byref(s), ctypes.byref(m))
    return s.value, m.value


def philox(ctr, key):
    c = (ctypes.c_uint32 * 4)(*ctr)
    k = (ctypes.c_uint32 * 2)(*key)
    o = (ctypes.c_uint32 * 4)()
    lib().orc_philox4x32_10(c, k, o)
    return list(o)


def normal(n: int, seed: int, stream: int, scale: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_normal(_f(out), n, seed, stream, scale)
    return out


def bytes_per_row(quant: int, head_dim: int) -> int:
    return lib().orc_bytes_per_row(quant, head_dim)


# ---------------------------------------------------------------- q/k preparation
def rope_tables(n_rot: int, max_pos: int, theta: float):
    """RotaryEmbedding::new tables (qwen3_next.rs:878-904): cos, sin [max_pos, n_rot/2]."""
    half = n_rot // 2
    c = np.zeros((max_pos, half), dtype=np.float32)
    s = np.zeros((max_pos, half), dtype=np.float32)
    rc = lib().orc_rope_tables(n_rot, max_pos, theta, _f(c), _f(s))
    if rc != OK:
        raise ValueError(f"orc_rope_tables failed ({rc})")
    return c, s


def rms_norm(x: np.ndarray, alpha: np.ndarray, eps: float) -> np.ndarray:
    """candle_nn::ops::rms_norm over the last axis (qwen3_next.rs:2369, 2389)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    a = np.ascontiguousarray(alpha, dtype=np.float32)
    d = x.shape[-1]
    y = np.empty_like(x)
    lib().orc_rms_norm(_f(x), _f(a), eps, x.size // d, d, _f(y))
    return y


def rope_rows(x: np.ndarray, pos: np.ndarray, n_rot: int, cos: np.ndarray,
              sin: np.ndarray) -> np.ndarray:
    """candle rope on x[..., :n_rot]; pos gives each row's position (flattened rows)."""
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    d = y.shape[-1]
    p = np.ascontiguousarray(pos, dtype=np.int64).reshape(-1)
    assert p.size == y.size // d
    rc = lib().orc_rope_rows(_f(y), p.size, d, n_rot, p.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                             _f(np.ascontiguousarray(cos)), _f(np.ascontiguousarray(sin)))
    if rc != OK:
        raise ValueError(f"orc_rope_rows failed ({rc})")
    return y


def qk_prep(q, k, q_alpha, k_alpha, eps: float, n_rot: int, cos, sin, offset: int):
    """q [b, l, H, d], k [b, l, Hkv, d] -> (q_norm + rope, k_norm + rope) at positions
    offset + t (FullAttention::forward, qwen3_next.rs:2369-2399). Either may be None."""
    ref = q if q is not None else k
    b, l, _, d = ref.shape
    qa = np.ascontiguousarray(q, dtype=np.float32) if q is not None else None
    ka = np.ascontiguousarray(k, dtype=np.float32) if k is not None else None
    qo = np.empty_like(qa) if qa is not None else None
    ko = np.empty_like(ka) if ka is not None else None
    nul = ctypes.cast(None, _fp)
    rc = lib().orc_qk_prep(
        _f(qa) if qa is not None else nul, _f(ka) if ka is not None else nul, b, l,
        qa.shape[2] if qa is not None else 0, ka.shape[2] if ka is not None else 0, d,
        _f(np.ascontiguousarray(q_alpha, dtype=np.float32)) if qa is not None else nul,
        _f(np.ascontiguousarray(k_alpha, dtype=np.float32)) if ka is not None else nul,
        eps, n_rot, _f(np.ascontiguousarray(cos)), _f(np.ascontiguousarray(sin)), offset,
        _f(qo) if qo is not None else nul, _f(ko) if ko is not None else nul)
    if rc != OK:
        raise ValueError(f"orc_qk_prep failed ({rc})")
    return qo, ko


# ---------------------------------------------------------------- cache
class Cache:
    """CPU restatement of PreallocatedQuantizedKvCache (qwen3_next.rs:343-643)."""

    def __init__(self, quant: int, batch: int, n_kv_heads: int, head_dim: int, max_seq_len: int):
        self._c = OrcCache()
        rc = lib().orc_cache_init(ctypes.byref(self._c), quant, batch, n_kv_heads, head_dim,
                                  max_seq_len)
        if rc != OK:
            raise ValueError(f"orc_cache_init failed ({rc})")

    def __del__(self):
        try:
            lib().orc_cache_free(ctypes.byref(self._c))
        except Exception:
            pass

    @property
    def seq_len(self) -> int:
        return self._c.seq_len

    @property
    def bytes_per_row(self) -> int:
        return self._c.bytes_per_row

    def _shape_ok(self, k: np.ndarray):
        c = self._c
        assert k.shape[0] == c.batch and k.shape[1] == c.n_kv_heads and k.shape[3] == c.head_dim

    def append(self, k: np.ndarray, v: np.ndarray) -> int:
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        self._shape_ok(k)
        return lib().orc_cache_append(ctypes.byref(self._c), _f(k), _f(v), k.shape[2])

    def append_at(self, k: np.ndarray, v: np.ndarray, offset: int) -> int:
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        self._shape_ok(k)
        return lib().orc_cache_append_at(ctypes.byref(self._c), _f(k), _f(v), k.shape[2], offset)

    def truncate(self, n: int) -> None:
        lib().orc_cache_truncate(ctypes.byref(self._c), n)

    def clear(self) -> None:
        lib().orc_cache_clear(ctypes.byref(self._c))

    def resize_batch(self, b: int) -> int:
        return lib().orc_cache_resize_batch(ctypes.byref(self._c), b)

    def valid_bytes(self):
        """(k_bytes, v_bytes) over [0, seq_len) rows, seq-major."""
        c = self._c
        n = c.seq_len * c.batch * c.n_kv_heads * c.bytes_per_row
        k = np.ctypeslib.as_array(c.k, shape=(max(n, 1),))[:n].copy()
        v = np.ctypeslib.as_array(c.v, shape=(max(n, 1),))[:n].copy()
        return k, v

    def load_bytes(self, k: np.ndarray, v: np.ndarray, seq_len: int) -> None:
        """Overwrite rows [0, seq_len) with given packed bytes (e.g. read back from a GPU)."""
        c = self._c
        n = seq_len * c.batch * c.n_kv_heads * c.bytes_per_row
        assert seq_len <= c.max_seq_len and k.size >= n and v.size >= n
        k = np.ascontiguousarray(k, dtype=np.uint8)
        v = np.ascontiguousarray(v, dtype=np.uint8)
        ctypes.memmove(c.k, k.ctypes.data, n)
        ctypes.memmove(c.v, v.ctypes.data, n)
        c.seq_len = seq_len

    def get_kv(self):
        c = self._c
        shape = (c.batch, c.n_kv_heads, c.seq_len, c.head_dim)
        k = np.zeros(shape, dtype=np.float32)
        v = np.zeros(shape, dtype=np.float32)
        lib().orc_cache_get_kv(ctypes.byref(self._c), _f(k), _f(v))
        return k, v

    def attend(self, q: np.ndarray, scale: float, q_offset: int, causal: bool,
               mode: str = "f32", threads: int = 0) -> np.ndarray:
        q = np.ascontiguousarray(q, dtype=np.float32)
        b, l, H, d = q.shape
        if mode == "f64":
            out = np.zeros(q.shape, dtype=np.float64)
            rc = lib().orc_attend_f64(ctypes.byref(self._c), _f(q), l, H, scale, q_offset,
                                      int(causal), out.ctypes.data_as(_dp))
        else:
            out = np.zeros(q.shape, dtype=np.float32)
            fn = lib().orc_attend_f32 if mode == "f32" else lib().orc_attend_faithful
            rc = fn(ctypes.byref(self._c), _f(q), l, H, scale, q_offset, int(causal), _f(out),
                    threads)
        if rc != OK:
            raise ValueError(f"oracle attend failed ({rc})")
        return out


def deltanet_step(q, k, v, gate, beta, state, gate_offset, scale: float, eps: float):
    """orc_deltanet_step on numpy arrays: q, k, v [b, h, d]; gate, beta [b, h]; state
    [b, h, d, d] (v index, k index) and gate_offset [b, h] (or None) updated in place.
    Returns out [b, h, d]."""
    b, h, d = q.shape
    for a in (q, k, v, gate, beta, state) + ((gate_offset,) if gate_offset is not None else ()):
        assert a.dtype == np.float32 and a.flags.c_contiguous
    assert state.shape == (b, h, d, d) and gate.shape == (b, h) and beta.shape == (b, h)
    out = np.empty_like(v)
    lib().orc_deltanet_step(_f(q), _f(k), _f(v), _f(gate), _f(beta), _f(state),
                            _f(gate_offset) if gate_offset is not None else None, _f(out),
                            b, h, d, scale, eps)
    return out


# GGUF weight types of the output projection (GGML's ggml_type numbers)
W_Q8_0, W_Q4K, W_Q5K, W_Q6K = 8, 12, 13, 14
W_BLOCK = {W_Q8_0: 32, W_Q4K: 256, W_Q5K: 256, W_Q6K: 256}
W_BLOCK_BYTES = {W_Q8_0: 34, W_Q4K: 144, W_Q5K: 176, W_Q6K: 210}


def dequantize_weight(b: np.ndarray, w_type: int, n: int) -> np.ndarray:
    """orc_{q8_0,q4k,q5k,q6k}_dequantize of n elements of GGUF type w_type."""
    b = np.ascontiguousarray(b, dtype=np.uint8)
    assert b.size >= n // W_BLOCK[w_type] * W_BLOCK_BYTES[w_type]
    y = np.zeros(n, dtype=np.float32)
    fn = {W_Q8_0: lib().orc_q8_0_dequantize, W_Q4K: lib().orc_q4k_dequantize,
          W_Q5K: lib().orc_q5k_dequantize, W_Q6K: lib().orc_q6k_dequantize}[w_type]
    fn(_u8(b), _f(y), n)
    return y


def gated_oproj(attn, gate, w_bytes, w_type: int, out_dim: int):
    """orc_gated_oproj: attn, gate [b, in_dim] f32 (gate None: no gating), w_bytes the uint8
    rows of GGUF type w_type [out_dim * row bytes]. Returns [b, out_dim]."""
    b, in_dim = attn.shape
    assert w_bytes.size == out_dim * lib().orc_weight_row_bytes(w_type, in_dim)
    out = np.empty((b, out_dim), np.float32)
    rc = lib().orc_gated_oproj(_f(attn), _f(gate) if gate is not None else None, _u8(w_bytes),
                               w_type, _f(out), b, in_dim, out_dim)
    assert rc == 0, rc
    return out


def gated_oproj_q4k(attn, gate, w_bytes, out_dim: int):
    """orc_gated_oproj_q4k: attn, gate [b, in_dim] f32 (gate None: no gating), w_bytes the
    uint8 Q4K rows [out_dim * in_dim / 256 * 144]. Returns [b, out_dim]."""
    b, in_dim = attn.shape
    assert w_bytes.size == out_dim * (in_dim // 256) * 144
    out = np.empty((b, out_dim), np.float32)
    lib().orc_gated_oproj_q4k(_f(attn), _f(gate) if gate is not None else None, _u8(w_bytes),
                              _f(out), b, in_dim, out_dim)
    return out
