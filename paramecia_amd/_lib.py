"""ctypes binding of libpkv.so (include/pkv.h).

There is no fallback: if the HIP library is missing the import of any entry point
raises, so a GPU run can never silently fall back to CPU code.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpkv.so")

QUANT_NONE, QUANT_F16, QUANT_BF16, QUANT_Q8_0, QUANT_Q4K = 0, 1, 2, 3, 4
OK, ERR_OVERFLOW, ERR_OFFSET, ERR_ARG, ERR_HIP, ERR_EMPTY, ERR_LAYERS, ERR_LAYOUT, \
    ERR_UNSUPPORTED = range(9)
ENTRY_EMPTY, ENTRY_FULL, ENTRY_LINEAR = 0, 1, 2
RESTORE_BYTES, RESTORE_REQUANTIZE = 0, 1

# Every exported symbol of include/pkv.h (checked by tests/test_abi.py).
SYMBOLS = (
    "pkv_last_error", "pkv_version", "pkv_device_status", "pkv_quant_parse", "pkv_quant_default",
    "pkv_quant_block_size", "pkv_quant_is_ggml", "pkv_bytes_per_row", "pkv_create",
    "pkv_destroy", "pkv_set_stream", "pkv_len", "pkv_capacity", "pkv_geometry",
    "pkv_truncate", "pkv_set_len", "pkv_clear", "pkv_resize_batch", "pkv_append", "pkv_attend",
    "pkv_append_attend", "pkv_get_kv", "pkv_kv_storage", "pkv_flash_attn", "pkv_flash_attn_noalloc",
    "pkv_append_attend_batched", "pkv_prefix_create", "pkv_prefix_free", "pkv_prefix_tokens",
    "pkv_prefix_num_layers", "pkv_prefix_entry_kind", "pkv_prefix_save_full",
    "pkv_prefix_save_linear", "pkv_prefix_linear_sizes", "pkv_prefix_full_len",
    "pkv_prefix_restore", "pkv_fill_normal", "pkv_scale_channels", "pkv_copy_segments",
    "pkv_rope_tables_host", "pkv_rope_create", "pkv_rope_destroy", "pkv_rope_geometry",
    "pkv_append_prep", "pkv_append_attend_prep", "pkv_deltanet_step",
    "pkv_gated_oproj_q4k", "pkv_gated_oproj", "pkv_prefix_serialized_size", "pkv_prefix_serialize",
    "pkv_prefix_deserialize", "pkv_pool_create", "pkv_pool_destroy", "pkv_pool_free_pages",
    "pkv_pool_set_stream", "pkv_seq_create", "pkv_seq_destroy", "pkv_seq_len", "pkv_seq_pages",
    "pkv_seq_fork", "pkv_seq_truncate", "pkv_seq_append", "pkv_seq_attend",
    "pkv_seq_decode_batched", "pkv_seq_get_kv", "pkv_seq_append_batched",
    "pkv_seq_append_decode_batched",
)


class PkvError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[pkv {code}] {msg}")
        self.code = code


class LayerTarget(ctypes.Structure):
    _fields_ = [
        ("cache", ctypes.c_void_p),
        ("ssm", ctypes.c_void_p),
        ("conv", ctypes.c_void_p),
        ("gate_offset", ctypes.c_void_p),
        ("state_valid", ctypes.POINTER(ctypes.c_int)),
        ("ssm_cap", ctypes.c_size_t),
        ("conv_cap", ctypes.c_size_t),
        ("gate_cap", ctypes.c_size_t),
    ]


class QkPrep(ctypes.Structure):
    """pkv_qk_prep: one layer's q_norm / k_norm alphas, eps and the shared rope."""
    _fields_ = [
        ("q_alpha", ctypes.c_void_p),
        ("k_alpha", ctypes.c_void_p),
        ("eps", ctypes.c_float),
        ("rope", ctypes.c_void_p),
    ]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built: run `python -c 'import __graft_entry__ as g; g.build()'`")
        L = ctypes.CDLL(LIB_PATH)
        _declare(L)
        _lib = L
    return _lib


def _declare(L: ctypes.CDLL) -> None:
    c_int, c_i64, c_u64, c_sz = ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_size_t
    vp, fl = ctypes.c_void_p, ctypes.c_float
    P = ctypes.POINTER
    sig = {
        "pkv_last_error": ([], ctypes.c_char_p),
        "pkv_version": ([], ctypes.c_char_p),
        "pkv_device_status": ([], c_int),
        "pkv_quant_parse": ([ctypes.c_char_p, P(c_int)], c_int),
        "pkv_quant_default": ([], c_int),
        "pkv_quant_block_size": ([c_int], c_int),
        "pkv_quant_is_ggml": ([c_int], c_int),
        "pkv_bytes_per_row": ([c_int, c_int], c_sz),
        "pkv_create": ([c_int, c_int, c_int, c_int, c_i64, vp, P(vp)], c_int),
        "pkv_destroy": ([vp], c_int),
        "pkv_set_stream": ([vp, vp], c_int),
        "pkv_len": ([vp], c_i64),
        "pkv_capacity": ([vp], c_i64),
        "pkv_geometry": ([vp, P(c_int), P(c_int), P(c_int), P(c_int), P(c_sz)], c_int),
        "pkv_truncate": ([vp, c_i64], c_int),
        "pkv_set_len": ([vp, c_i64], c_int),
        "pkv_clear": ([vp], c_int),
        "pkv_resize_batch": ([vp, c_int], c_int),
        "pkv_append": ([vp, vp, vp, c_i64, c_i64], c_int),
        "pkv_attend": ([vp, vp, c_int, c_int, fl, c_i64, c_int, vp], c_int),
        "pkv_append_attend": ([vp, vp, vp, vp, c_int, fl, c_i64, vp], c_int),
        "pkv_get_kv": ([vp, vp, vp], c_int),
        "pkv_kv_storage": ([vp, P(vp), P(vp), P(c_sz), P(c_i64)], c_int),
        "pkv_flash_attn": ([c_int, vp, vp, vp, P(c_i64), fl, c_int, c_int, c_int, c_int, c_int,
                            c_i64, c_i64, c_int, vp, vp], c_int),
        "pkv_flash_attn_noalloc": ([c_int, vp, vp, vp, P(c_i64), fl, c_int, c_int, c_int, c_int,
                                    c_int, c_i64, c_i64, c_int, vp, vp], c_int),
        "pkv_append_attend_batched": ([P(vp), c_int, vp, vp, vp, c_int, fl, vp, vp], c_int),
        "pkv_prefix_create": ([P(ctypes.c_uint32), c_sz, c_int, P(vp)], c_int),
        "pkv_prefix_free": ([vp], c_int),
        "pkv_prefix_tokens": ([vp, P(P(ctypes.c_uint32)), P(c_sz)], c_int),
        "pkv_prefix_num_layers": ([vp], c_int),
        "pkv_prefix_entry_kind": ([vp, c_int], c_int),
        "pkv_prefix_save_full": ([vp, c_int, vp], c_int),
        "pkv_prefix_save_linear": ([vp, c_int, vp, c_sz, vp, c_sz, vp, c_sz, vp], c_int),
        "pkv_prefix_linear_sizes": ([vp, c_int, P(c_sz), P(c_sz), P(c_sz)], c_int),
        "pkv_prefix_full_len": ([vp, c_int], c_i64),
        "pkv_prefix_restore": ([vp, P(LayerTarget), c_int, c_int, P(c_sz), vp], c_int),
        "pkv_fill_normal": ([vp, c_sz, c_u64, c_u64, fl, vp], c_int),
        "pkv_scale_channels": ([vp, c_sz, c_int, P(c_int), c_int, fl, vp], c_int),
        "pkv_copy_segments": ([P(vp), P(vp), P(c_sz), c_int, vp], c_int),
        "pkv_rope_tables_host": ([c_int, c_i64, ctypes.c_double, vp, vp], c_int),
        "pkv_rope_create": ([c_int, c_i64, ctypes.c_double, P(vp)], c_int),
        "pkv_rope_destroy": ([vp], c_int),
        "pkv_rope_geometry": ([vp, P(c_int), P(c_i64), P(vp), P(vp)], c_int),
        "pkv_append_prep": ([vp, P(QkPrep), vp, c_int, vp, vp, vp, c_i64, c_i64], c_int),
        "pkv_append_attend_prep": ([vp, P(QkPrep), vp, vp, vp, c_int, fl, c_i64, vp], c_int),
        "pkv_deltanet_step": ([vp] * 8 + [c_int] * 3 + [fl, fl, vp], c_int),
        "pkv_gated_oproj_q4k": ([vp] * 4 + [c_int] * 3 + [vp], c_int),
        "pkv_gated_oproj": ([vp] * 3 + [c_int, vp] + [c_int] * 3 + [vp], c_int),
        "pkv_prefix_serialized_size": ([vp], c_sz),
        "pkv_prefix_serialize": ([vp, vp, c_sz, vp], c_int),
        "pkv_prefix_deserialize": ([vp, c_sz, P(vp), vp], c_int),
        "pkv_pool_create": ([c_int] * 5 + [vp, P(vp)], c_int),
        "pkv_pool_destroy": ([vp], c_int),
        "pkv_pool_free_pages": ([vp], c_int),
        "pkv_pool_set_stream": ([vp, vp], c_int),
        "pkv_seq_create": ([vp, P(vp)], c_int),
        "pkv_seq_destroy": ([vp], c_int),
        "pkv_seq_len": ([vp], c_i64),
        "pkv_seq_pages": ([vp], c_int),
        "pkv_seq_fork": ([vp, P(vp)], c_int),
        "pkv_seq_truncate": ([vp, c_i64], c_int),
        "pkv_seq_append": ([vp, vp, vp, c_i64, c_i64], c_int),
        "pkv_seq_attend": ([vp, vp, c_int, c_int, fl, c_i64, c_int, vp], c_int),
        "pkv_seq_decode_batched": ([P(vp), c_int, vp, c_int, fl, vp], c_int),
        "pkv_seq_get_kv": ([vp, vp, vp], c_int),
        "pkv_seq_append_batched": ([P(vp), c_int, vp, vp], c_int),
        "pkv_seq_append_decode_batched": ([P(vp), c_int, vp, vp, vp, c_int, fl, vp], c_int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res


def check(rc: int) -> None:
    if rc != OK:
        raise PkvError(rc, lib().pkv_last_error().decode())
