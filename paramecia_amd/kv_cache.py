"""Host-side mirror of paramecia-model's KV-cache API on top of libpkv.

Names, argument meaning and error behaviour follow the reference
(paramecia-model/src/qwen3_next.rs): KvCacheQuantization (:88-166),
PreallocatedQuantizedKvCache (:343-643), the cache block of FullAttention::forward
(:2401-2561), RecurrentState / PrefixCacheEntry / PrefixCache (:683-864) and the
ModelWeights cache methods (:5466-5501, :5685-5750). Tensors are torch device tensors;
torch provides memory and streams only, every kernel is libpkv's.
"""
from __future__ import annotations

import ctypes
import json
import struct
import enum
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import torch

from . import _lib
from ._lib import PkvError, check, lib


# ------------------------------------------------------------------ errors
class KvCacheError(RuntimeError):
    """candle::bail! on the KV-cache path."""


class KvCacheOverflow(KvCacheError):
    pass


class KvCacheOffsetMismatch(KvCacheError):
    pass


class EmptyCacheError(KvCacheError):
    pass


class PrefixLayerMismatch(KvCacheError):
    pass


_ERRORS = {
    _lib.ERR_OVERFLOW: KvCacheOverflow,
    _lib.ERR_OFFSET: KvCacheOffsetMismatch,
    _lib.ERR_EMPTY: EmptyCacheError,
    _lib.ERR_LAYERS: PrefixLayerMismatch,
}


def np_prod(shape) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    return n


def _call(rc: int) -> None:
    if rc != _lib.OK:
        msg = lib().pkv_last_error().decode()
        raise _ERRORS.get(rc, KvCacheError)(f"[pkv {rc}] {msg}")


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _f32(t: torch.Tensor, name: str) -> torch.Tensor:
    if not t.is_cuda or t.dtype != torch.float32:
        raise KvCacheError(f"{name} must be a float32 device tensor")
    return t.contiguous()


class _DeviceBytes:
    """__cuda_array_interface__ view of library-owned device bytes."""

    def __init__(self, ptr: int, n: int):
        self.__cuda_array_interface__ = {
            "shape": (n,), "typestr": "|u1", "data": (ptr, False), "version": 3,
            "strides": None,
        }


# ------------------------------------------------------------------ KvCacheQuantization
class KvCacheQuantization(enum.IntEnum):
    NONE = _lib.QUANT_NONE  # deprecated alias of F16
    F16 = _lib.QUANT_F16
    BF16 = _lib.QUANT_BF16
    Q8_0 = _lib.QUANT_Q8_0
    Q4K = _lib.QUANT_Q4K

    @classmethod
    def default(cls) -> "KvCacheQuantization":
        return cls(lib().pkv_quant_default())

    @classmethod
    def from_str(cls, s: str) -> Optional["KvCacheQuantization"]:
        out = ctypes.c_int()
        rc = lib().pkv_quant_parse(s.encode(), ctypes.byref(out))
        return cls(out.value) if rc == _lib.OK else None

    def block_size(self) -> int:
        return lib().pkv_quant_block_size(int(self))

    def to_ggml_dtype(self) -> Optional[str]:
        return {KvCacheQuantization.Q8_0: "Q8_0", KvCacheQuantization.Q4K: "Q4K"}.get(self)

    def cache_dtype(self) -> Optional[torch.dtype]:
        if self in (KvCacheQuantization.NONE, KvCacheQuantization.F16):
            return torch.float16
        if self == KvCacheQuantization.BF16:
            return torch.bfloat16
        return None


# ------------------------------------------------------------------ the cache
class PreallocatedQuantizedKvCache:
    """Device-resident preallocated cache with O(1) append and quantize-on-write."""

    def __init__(self, batch_size: int, num_kv_heads: int, max_seq_len: int, head_dim: int,
                 quant: KvCacheQuantization = KvCacheQuantization.Q4K, stream: Optional[int] = None):
        h = ctypes.c_void_p()
        _call(lib().pkv_create(int(quant), batch_size, num_kv_heads, head_dim, max_seq_len,
                               ctypes.c_void_p(stream if stream is not None else _stream()),
                               ctypes.byref(h)))
        self._h = h
        self._lib = lib()  # held for __del__, which may run during interpreter shutdown
        self._stream = stream if stream is not None else _stream()
        self.quant = KvCacheQuantization(int(quant) or _lib.QUANT_F16)
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.bytes_per_row = lib().pkv_bytes_per_row(int(quant), head_dim)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.pkv_destroy(h)
            self._h = None

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    @property
    def seq_len(self) -> int:
        return lib().pkv_len(self._h)

    @property
    def max_seq_len(self) -> int:
        """Capacity in tokens. Q8_0/Q4K caches keep it; F16/BF16 caches grow past it on an
        append (the reference's float cache grows by Tensor::cat, qwen3_next.rs:2492-2516)."""
        return lib().pkv_capacity(self._h)

    @property
    def batch_size(self) -> int:
        b = ctypes.c_int()
        check(lib().pkv_geometry(self._h, None, ctypes.byref(b), None, None, None))
        return b.value

    def set_stream(self, stream: int) -> None:
        check(lib().pkv_set_stream(self._h, ctypes.c_void_p(stream)))
        self._stream = stream

    def _follow_stream(self) -> None:
        """Work is enqueued on torch's current stream (so graph capture sees it)."""
        s = _stream()
        if s != self._stream:
            self.set_stream(s)

    def append_quantized(self, new_k: torch.Tensor, new_v: torch.Tensor,
                         offset: int = -1) -> None:
        """new_k, new_v: [batch, num_kv_heads, n, head_dim] f32 (qwen3_next.rs:431)."""
        self._follow_stream()
        k, v = _f32(new_k, "new_k"), _f32(new_v, "new_v")
        if k.shape != v.shape or k.dim() != 4:
            raise KvCacheError("new_k/new_v must both be [batch, heads, n, head_dim]")
        _call(lib().pkv_append(self._h, _ptr(k), _ptr(v), k.shape[2], offset))

    def append(self, new_k: torch.Tensor, new_v: torch.Tensor):
        self.append_quantized(new_k, new_v)
        return self.get_kv()

    def get_kv(self):
        """Dequantized [batch, heads, seq_len, head_dim] f32 tensors (qwen3_next.rs:520)."""
        self._follow_stream()
        shape = (self.batch_size, self.num_kv_heads, self.seq_len, self.head_dim)
        k = torch.empty(shape, dtype=torch.float32, device="cuda")
        v = torch.empty(shape, dtype=torch.float32, device="cuda")
        _call(lib().pkv_get_kv(self._h, _ptr(k), _ptr(v)))
        return k, v

    def get_kv_storage(self):
        """(k_ptr, v_ptr, valid_bytes, (stride_b, stride_seq, stride_h, stride_d))."""
        kp, vp, n = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_size_t()
        st = (ctypes.c_int64 * 4)()
        _call(lib().pkv_kv_storage(self._h, ctypes.byref(kp), ctypes.byref(vp), ctypes.byref(n), st))
        return kp.value, vp.value, n.value, tuple(st)

    def raw_bytes(self):
        """Copies of the valid packed K and V bytes as uint8 device tensors."""
        if self.seq_len == 0:
            e = torch.empty(0, dtype=torch.uint8, device="cuda")
            return e, e.clone()
        kp, vp, n, _ = self.get_kv_storage()
        k = torch.as_tensor(_DeviceBytes(kp, n), device="cuda").clone()
        v = torch.as_tensor(_DeviceBytes(vp, n), device="cuda").clone()
        return k, v

    def attend(self, q: torch.Tensor, scale: float, q_offset: int, causal: bool = True) -> torch.Tensor:
        """q: [batch, l, num_heads, head_dim] f32 -> out of the same shape."""
        self._follow_stream()
        q = _f32(q, "q")
        out = torch.empty_like(q)
        _call(lib().pkv_attend(self._h, _ptr(q), q.shape[1], q.shape[2], scale, q_offset,
                               int(causal), _ptr(out)))
        return out

    def append_attend(self, new_k, new_v, q, scale: float, offset: int = -1) -> torch.Tensor:
        """Fused decode step: append one token and attend over every key."""
        self._follow_stream()
        k, v, q = _f32(new_k, "new_k"), _f32(new_v, "new_v"), _f32(q, "q")
        out = torch.empty_like(q)
        _call(lib().pkv_append_attend(self._h, _ptr(k), _ptr(v), _ptr(q), q.shape[2], scale,
                                      offset, _ptr(out)))
        return out

    def append_prep(self, q: Optional[torch.Tensor], new_k: torch.Tensor, new_v: torch.Tensor,
                    prep: "QkPrep", offset: int = -1) -> Optional[torch.Tensor]:
        """q_norm / k_norm, rope and append_quantized in one launch (qwen3_next.rs:2369-2442).
        q: [batch, n, num_heads, d] or None; new_k, new_v: [batch, n, num_kv_heads, d], the
        projection outputs before the transpose. Returns the prepared q (same layout)."""
        self._follow_stream()
        k, v = _f32(new_k, "new_k"), _f32(new_v, "new_v")
        if k.shape != v.shape or k.dim() != 4:
            raise KvCacheError("new_k/new_v must both be [batch, n, heads, head_dim]")
        qq = _f32(q, "q") if q is not None else None
        q_out = torch.empty_like(qq) if qq is not None else None
        H = qq.shape[2] if qq is not None else 0
        _call(lib().pkv_append_prep(self._h, ctypes.byref(prep.c), _ptr(qq), H, _ptr(q_out),
                                    _ptr(k), _ptr(v), k.shape[1], offset))
        return q_out

    def append_attend_prep(self, q: torch.Tensor, new_k: torch.Tensor, new_v: torch.Tensor,
                           prep: "QkPrep", scale: float, offset: int = -1) -> torch.Tensor:
        """Decode step from the projection outputs: prepare q and k, append, attend.
        q: [batch, 1, num_heads, d]; new_k, new_v: [batch, 1, num_kv_heads, d]."""
        self._follow_stream()
        k, v, qq = _f32(new_k, "new_k"), _f32(new_v, "new_v"), _f32(q, "q")
        out = torch.empty_like(qq)
        _call(lib().pkv_append_attend_prep(self._h, ctypes.byref(prep.c), _ptr(qq), _ptr(k),
                                           _ptr(v), qq.shape[2], scale, offset, _ptr(out)))
        return out

    def clear(self) -> None:
        check(lib().pkv_clear(self._h))

    def truncate(self, new_len: int) -> None:
        check(lib().pkv_truncate(self._h, new_len))

    def set_len(self, seq_len: int) -> None:
        """Assign seq_len directly, as LayerWeights::restore_cache does (qn:4326-4337)."""
        _call(lib().pkv_set_len(self._h, seq_len))

    def resize_batch(self, batch_size: int) -> None:
        self._follow_stream()
        _call(lib().pkv_resize_batch(self._h, batch_size))


# ------------------------------------------------------------------ paged caches
class PagedKvPool:
    """Pages of KV rows for one layer, shared by many sequences (pkv_pool_*): the
    multi-sequence form of PreallocatedQuantizedKvCache (qwen3_next.rs:343-643) for a
    serving loop, where the reference keeps one preallocated cache per sequence
    (paramecia-llm/src/backend/local.rs:743-800)."""

    def __init__(self, num_kv_heads: int, head_dim: int, page_tokens: int, n_pages: int,
                 quant: KvCacheQuantization = KvCacheQuantization.Q4K,
                 stream: Optional[int] = None):
        h = ctypes.c_void_p()
        self._stream = stream if stream is not None else _stream()
        _call(lib().pkv_pool_create(int(quant), num_kv_heads, head_dim, page_tokens, n_pages,
                                    ctypes.c_void_p(self._stream), ctypes.byref(h)))
        self._h = h
        self._lib = lib()
        self.quant = KvCacheQuantization(int(quant) or _lib.QUANT_F16)
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.page_tokens = page_tokens
        self.n_pages = n_pages

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.pkv_pool_destroy(h)
            self._h = None

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    @property
    def free_pages(self) -> int:
        return lib().pkv_pool_free_pages(self._h)

    def _follow_stream(self) -> None:
        s = _stream()
        if s != self._stream:
            check(lib().pkv_pool_set_stream(self._h, ctypes.c_void_p(s)))
            self._stream = s

    def sequence(self) -> "PagedSequence":
        return PagedSequence(self)

    def append_batched(self, seqs: Sequence["PagedSequence"], new_k: torch.Tensor,
                       new_v: torch.Tensor) -> None:
        """One token per sequence: new_k, new_v [n, num_kv_heads, 1, head_dim] f32
        (pkv_seq_append_batched)."""
        self._follow_stream()
        k, v = _f32(new_k, "new_k"), _f32(new_v, "new_v")
        if k.shape != v.shape or k.dim() != 4 or k.shape[0] != len(seqs) or k.shape[2] != 1:
            raise KvCacheError("new_k/new_v must both be [n_sequences, heads, 1, head_dim]")
        arr = (ctypes.c_void_p * len(seqs))(*[sq.handle.value for sq in seqs])
        _call(lib().pkv_seq_append_batched(arr, len(seqs), _ptr(k), _ptr(v)))

    def decode_batched(self, seqs: Sequence["PagedSequence"], q: torch.Tensor,
                       scale: float) -> torch.Tensor:
        """One decode query per sequence: q [n, num_heads, head_dim] -> out of that shape,
        each sequence attending over all its keys (pkv_seq_decode_batched)."""
        self._follow_stream()
        q = _f32(q, "q")
        if q.dim() != 3 or q.shape[0] != len(seqs):
            raise KvCacheError("q must be [n_sequences, num_heads, head_dim]")
        out = torch.empty_like(q)
        arr = (ctypes.c_void_p * len(seqs))(*[sq.handle.value for sq in seqs])
        _call(lib().pkv_seq_decode_batched(arr, len(seqs), _ptr(q), q.shape[1], scale, _ptr(out)))
        return out

    def append_decode_batched(self, seqs: Sequence["PagedSequence"], new_k: torch.Tensor,
                              new_v: torch.Tensor, q: torch.Tensor, scale: float) -> torch.Tensor:
        """The fused decode step: one token appended to each sequence (new_k, new_v [n,
        num_kv_heads, 1, head_dim]) and one query per sequence over all its keys, the new
        one included (q [n, num_heads, head_dim] -> out of that shape;
        pkv_seq_append_decode_batched)."""
        self._follow_stream()
        k, v, q = _f32(new_k, "new_k"), _f32(new_v, "new_v"), _f32(q, "q")
        if k.shape != v.shape or k.dim() != 4 or k.shape[0] != len(seqs) or k.shape[2] != 1:
            raise KvCacheError("new_k/new_v must both be [n_sequences, heads, 1, head_dim]")
        if q.dim() != 3 or q.shape[0] != len(seqs):
            raise KvCacheError("q must be [n_sequences, num_heads, head_dim]")
        out = torch.empty_like(q)
        arr = (ctypes.c_void_p * len(seqs))(*[sq.handle.value for sq in seqs])
        _call(lib().pkv_seq_append_decode_batched(arr, len(seqs), _ptr(k), _ptr(v), _ptr(q),
                                                  q.shape[1], scale, _ptr(out)))
        return out


class PagedSequence:
    """One sequence of a PagedKvPool, with the cache API of PreallocatedQuantizedKvCache at
    batch 1 (append_quantized / attend / get_kv / truncate) plus fork (page sharing)."""

    def __init__(self, pool: PagedKvPool, _handle: Optional[ctypes.c_void_p] = None):
        self.pool = pool  # keeps the pool alive while the sequence lives
        self._lib = lib()
        if _handle is None:
            _handle = ctypes.c_void_p()
            _call(lib().pkv_seq_create(pool.handle, ctypes.byref(_handle)))
        self._h = _handle

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.pkv_seq_destroy(h)
            self._h = None

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    @property
    def seq_len(self) -> int:
        return lib().pkv_seq_len(self._h)

    @property
    def pages(self) -> int:
        return lib().pkv_seq_pages(self._h)

    def fork(self) -> "PagedSequence":
        h = ctypes.c_void_p()
        _call(lib().pkv_seq_fork(self._h, ctypes.byref(h)))
        return PagedSequence(self.pool, h)

    def append_quantized(self, new_k: torch.Tensor, new_v: torch.Tensor,
                         offset: int = -1) -> None:
        """new_k, new_v: [1, num_kv_heads, n, head_dim] f32."""
        self.pool._follow_stream()
        k, v = _f32(new_k, "new_k"), _f32(new_v, "new_v")
        if k.shape != v.shape or k.dim() != 4 or k.shape[0] != 1:
            raise KvCacheError("new_k/new_v must both be [1, heads, n, head_dim]")
        _call(lib().pkv_seq_append(self._h, _ptr(k), _ptr(v), k.shape[2], offset))

    def get_kv(self):
        """Dequantized [1, heads, seq_len, head_dim] f32 tensors."""
        self.pool._follow_stream()
        shape = (1, self.pool.num_kv_heads, self.seq_len, self.pool.head_dim)
        k = torch.empty(shape, dtype=torch.float32, device="cuda")
        v = torch.empty(shape, dtype=torch.float32, device="cuda")
        _call(lib().pkv_seq_get_kv(self._h, _ptr(k), _ptr(v)))
        return k, v

    def attend(self, q: torch.Tensor, scale: float, q_offset: int,
               causal: bool = True) -> torch.Tensor:
        """q: [1, l, num_heads, head_dim] f32 -> out of the same shape."""
        self.pool._follow_stream()
        q = _f32(q, "q")
        out = torch.empty_like(q)
        _call(lib().pkv_seq_attend(self._h, _ptr(q), q.shape[1], q.shape[2], scale, q_offset,
                                   int(causal), _ptr(out)))
        return out

    def truncate(self, new_len: int) -> None:
        _call(lib().pkv_seq_truncate(self._h, new_len))


def flash_attn(quant: KvCacheQuantization, q: torch.Tensor, k_ptr: int, v_ptr: int,
               strides: Sequence[int], scale: float, num_kv_heads: int, seq_k: int,
               q_offset: int, causal: bool) -> torch.Tensor:
    """ops::flash_attn_q8 (paramecia-model/src/ops.rs:756) over caller-owned packed rows."""
    q = _f32(q, "q")
    b, l, H, d = q.shape
    out = torch.empty_like(q)
    st = (ctypes.c_int64 * 3)(*strides[:3])
    _call(lib().pkv_flash_attn(int(quant), _ptr(q), ctypes.c_void_p(k_ptr), ctypes.c_void_p(v_ptr),
                               st, scale, b, H, num_kv_heads, d, l, seq_k, q_offset, int(causal),
                               _ptr(out), ctypes.c_void_p(_stream())))
    return out


def append_attend_batched(caches: Sequence[PreallocatedQuantizedKvCache], k: torch.Tensor,
                          v: torch.Tensor, q: torch.Tensor, scale: float) -> torch.Tensor:
    """One decode step over independent batch-1 sequences in one launch.
    k, v: [n, num_kv_heads, head_dim]; q: [n, num_heads, head_dim]."""
    k, v, q = _f32(k, "k"), _f32(v, "v"), _f32(q, "q")
    out = torch.empty_like(q)
    arr = (ctypes.c_void_p * len(caches))(*[c.handle.value for c in caches])
    _call(lib().pkv_append_attend_batched(arr, len(caches), _ptr(k), _ptr(v), _ptr(q), q.shape[1],
                                          scale, _ptr(out), ctypes.c_void_p(_stream())))
    return out


# GGUF weight types of the output projection (GGML's ggml_type numbers)
WTYPE_Q8_0, WTYPE_Q4K, WTYPE_Q5K, WTYPE_Q6K = 8, 12, 13, 14
_W_BLOCK = {WTYPE_Q8_0: (32, 34), WTYPE_Q4K: (256, 144), WTYPE_Q5K: (256, 176),
            WTYPE_Q6K: (256, 210)}


def gated_o_proj(attn_output: torch.Tensor, gate: Optional[torch.Tensor], wo: torch.Tensor,
                 out_dim: int, w_type: int = WTYPE_Q4K) -> torch.Tensor:
    """The attention's gated output projection (qwen3_next.rs:2657-2680): attn_output, gate
    [b, l, in_dim] f32 (gate None: no gating), wo the uint8 GGUF bytes of self.wo in GGUF
    type w_type (Q4K: [out_dim, in_dim / 256, 144]; Q5K 176 B, Q6K 210 B per 256 inputs;
    Q8_0 34 B per 32). Returns [b, l, out_dim] (pkv_gated_oproj)."""
    x = _f32(attn_output, "attn_output")
    g = _f32(gate, "gate") if gate is not None else None
    if g is not None and g.shape != x.shape:
        raise KvCacheError("gate must have the attention output's shape")
    if w_type not in _W_BLOCK:
        raise KvCacheError(f"unsupported weight type {w_type} (Q8_0 8, Q4K 12, Q5K 13, Q6K 14)")
    in_dim = x.shape[-1]
    rows = x.numel() // in_dim
    blk, nbytes = _W_BLOCK[w_type]
    if wo.dtype != torch.uint8 or wo.numel() != out_dim * (in_dim // blk) * nbytes:
        raise KvCacheError(f"wo must hold out_dim x in_dim / {blk} blocks of {nbytes} B")
    out = torch.empty(x.shape[:-1] + (out_dim,), dtype=torch.float32, device=x.device)
    _call(lib().pkv_gated_oproj(_ptr(x), _ptr(g), _ptr(wo.contiguous()), w_type, _ptr(out), rows,
                                in_dim, out_dim, torch.cuda.current_stream().cuda_stream))
    return out


def fill_normal(t: torch.Tensor, seed: int, stream_id: int, scale: float = 1.0) -> torch.Tensor:
    """Seeded synthetic data identical to the CPU oracle's generator."""
    t = _f32(t, "t")
    _call(lib().pkv_fill_normal(_ptr(t), t.numel(), seed, stream_id, scale,
                                ctypes.c_void_p(_stream())))
    return t


def scale_channels(t: torch.Tensor, channels: Sequence[int], factor: float) -> torch.Tensor:
    t = _f32(t, "t")
    arr = (ctypes.c_int * len(channels))(*channels)
    _call(lib().pkv_scale_channels(_ptr(t), t.numel() // t.shape[-1], t.shape[-1], arr,
                                   len(channels), factor, ctypes.c_void_p(_stream())))
    return t


# ------------------------------------------------------------------ q/k preparation
class RotaryEmbedding:
    """RotaryEmbedding (qwen3_next.rs:866-940): cos/sin tables [max_pos, n_rot/2] built on
    the host as RotaryEmbedding::new does, kept on the device, shared by every layer."""

    def __init__(self, n_rot: int, max_position_embeddings: int, rope_theta: float):
        h = ctypes.c_void_p()
        _call(lib().pkv_rope_create(n_rot, max_position_embeddings, rope_theta, ctypes.byref(h)))
        self._h = h
        self.n_rot, self.max_pos, self.theta = n_rot, max_position_embeddings, rope_theta

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            lib().pkv_rope_destroy(h)
            self._h = None

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    @staticmethod
    def host_tables(n_rot: int, max_pos: int, rope_theta: float):
        """(cos, sin) [max_pos, n_rot/2] CPU float32 tensors from the library's host code
        (no device work)."""
        half = max(n_rot // 2, 1)
        c = torch.zeros((max_pos, half), dtype=torch.float32)
        s = torch.zeros((max_pos, half), dtype=torch.float32)
        _call(lib().pkv_rope_tables_host(n_rot, max_pos, rope_theta,
                                         ctypes.c_void_p(c.data_ptr()),
                                         ctypes.c_void_p(s.data_ptr())))
        return c, s

    def tables(self):
        """The device tables as [max_pos, n_rot/2] float32 tensors (copies)."""
        cp, sp = ctypes.c_void_p(), ctypes.c_void_p()
        _call(lib().pkv_rope_geometry(self._h, None, None, ctypes.byref(cp), ctypes.byref(sp)))
        n = self.max_pos * (self.n_rot // 2) * 4
        shape = (self.max_pos, self.n_rot // 2)
        c = torch.as_tensor(_DeviceBytes(cp.value, n), device="cuda").clone().view(torch.float32)
        s = torch.as_tensor(_DeviceBytes(sp.value, n), device="cuda").clone().view(torch.float32)
        return c.view(shape), s.view(shape)


class QkPrep:
    """One full-attention layer's q_norm / k_norm (RmsNorm alphas attn_q_norm.weight /
    attn_k_norm.weight, qwen3_next.rs:2297-2306) and the shared rope."""

    def __init__(self, q_alpha: torch.Tensor, k_alpha: torch.Tensor, eps: float,
                 rope: RotaryEmbedding):
        self.q_alpha = _f32(q_alpha, "q_alpha")
        self.k_alpha = _f32(k_alpha, "k_alpha")
        self.rope = rope
        self.eps = float(eps)
        self.c = _lib.QkPrep(self.q_alpha.data_ptr(), self.k_alpha.data_ptr(), self.eps,
                             rope.handle.value)


# ------------------------------------------------------------------ FullAttention's cache block
class FullAttentionKv:
    """The KV-cache half of FullAttention::forward (qwen3_next.rs:2401-2561): lazy cache
    creation, the offset rule (smaller offset truncates, larger errors), append, then
    causal GQA attention with q_offset = seq_len - l and scale 1/sqrt(head_dim)."""

    def __init__(self, num_heads: int, num_kv_heads: int, head_dim: int, max_seq_len: int,
                 quant: KvCacheQuantization = KvCacheQuantization.Q4K):
        self.num_heads, self.num_kv_heads, self.head_dim = num_heads, num_kv_heads, head_dim
        self.max_seq_len = max_seq_len
        self.kv_cache_quantization = quant
        self.quantized_cache: Optional[PreallocatedQuantizedKvCache] = None
        self.scale = float(1.0 / (head_dim ** 0.5))

    def _ensure(self, b: int) -> PreallocatedQuantizedKvCache:
        if self.quantized_cache is None:
            self.quantized_cache = PreallocatedQuantizedKvCache(
                b, self.num_kv_heads, self.max_seq_len, self.head_dim, self.kv_cache_quantization)
        return self.quantized_cache

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, offset: int) -> torch.Tensor:
        """q: [b, l, num_heads, d]; k, v: [b, num_kv_heads, l, d]. Returns [b, l, num_heads*d]."""
        b, l = q.shape[0], q.shape[1]
        cache = self._ensure(b)
        if l == 1:
            out = cache.append_attend(k, v, q, self.scale, offset)
        else:
            cache.append_quantized(k, v, offset)
            seq_k = cache.seq_len
            out = cache.attend(q, self.scale, seq_k - l, causal=True)
        return out.reshape(b, l, self.num_heads * self.head_dim)

    def forward_projected(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, offset: int,
                          prep: QkPrep) -> torch.Tensor:
        """From the projection outputs (qwen3_next.rs:2369-2561): q [b, l, num_heads, d],
        k, v [b, l, num_kv_heads, d], before q_norm / k_norm / rope. Returns [b, l, H*d]."""
        b, l = q.shape[0], q.shape[1]
        cache = self._ensure(b)
        if l == 1:
            out = cache.append_attend_prep(q, k, v, prep, self.scale, offset)
        else:
            qp = cache.append_prep(q, k, v, prep, offset)
            seq_k = cache.seq_len
            out = cache.attend(qp, self.scale, seq_k - l, causal=True)
        return out.reshape(b, l, self.num_heads * self.head_dim)

    def cache_seq_len(self) -> int:
        return 0 if self.quantized_cache is None else self.quantized_cache.seq_len

    def clear_kv_cache(self) -> None:
        if self.quantized_cache is not None:
            self.quantized_cache.clear()

    def truncate_kv_cache(self, new_len: int) -> None:
        if self.quantized_cache is not None:
            self.quantized_cache.truncate(new_len)

    def _is_float_cache(self) -> bool:
        c = self.quantized_cache
        return c is not None and c.quant in (KvCacheQuantization.F16, KvCacheQuantization.BF16)

    def checkpoint(self) -> "LayerCheckpoint":
        """LayerWeights::checkpoint_cache for a full-attention layer (qn:4311-4322): the
        reference records preallocated_cache.seq_len, and that field holds only the F16 /
        BF16 cache; a Q8_0 / Q4K cache lives in quantized_cache, so its checkpoint records 0."""
        return LayerCheckpoint("FullAttention", self.quantized_cache.seq_len if self._is_float_cache() else 0)

    def restore(self, seq_len: int) -> None:
        """LayerWeights::restore_cache (qn:4326-4337): assigns seq_len to the F16 / BF16 cache;
        a quantized cache is left as it is (the reference's preallocated_cache is None then)."""
        if self._is_float_cache():
            self.quantized_cache.set_len(seq_len)


@dataclass
class LayerCheckpoint:
    """LayerCheckpoint (qwen3_next.rs:827-832): FullAttention { seq_len } or the
    LinearAttention marker (the state sits in the layer's backup buffers)."""
    kind: str
    seq_len: int = 0


def _copy_segments(pairs) -> None:
    """Device copies dst <- src of equal-sized tensors, all in one libpkv launch."""
    n = len(pairs)
    if n == 0:
        return
    dst = (ctypes.c_void_p * n)(*[d.data_ptr() for d, _ in pairs])
    src = (ctypes.c_void_p * n)(*[x.data_ptr() for _, x in pairs])
    nb = (ctypes.c_size_t * n)(*[x.numel() * x.element_size() for _, x in pairs])
    _call(lib().pkv_copy_segments(dst, src, nb, n, ctypes.c_void_p(_stream())))


def _reuse(spare: Optional[torch.Tensor], like: torch.Tensor) -> torch.Tensor:
    if spare is not None and spare.shape == like.shape and spare.dtype == like.dtype:
        return spare
    return torch.empty_like(like, memory_format=torch.contiguous_format)


@dataclass
class RecurrentState:
    """Gated-DeltaNet state of one linear-attention layer (qwen3_next.rs:683-700), with the
    checkpoint / restore backups of speculative decoding (:733-757)."""
    ssm_state: torch.Tensor             # [b, heads, dk, dv] f32
    conv_state: torch.Tensor            # [b, conv_dim, kernel-1] f32
    gate_cumsum_offset: Optional[torch.Tensor] = None  # [b, heads] f32
    backup_ssm: Optional[torch.Tensor] = None
    backup_conv: Optional[torch.Tensor] = None
    backup_gate_offset: Optional[torch.Tensor] = None
    _spare: list = field(default_factory=lambda: [None, None, None], repr=False)

    def checkpoint(self) -> None:
        """RecurrentState::checkpoint (qn:733-744). The reference keeps shallow clones
        because its steps replace the state tensors; pkv_deltanet_step updates them in
        place, so the backups are copies, made in one launch into buffers kept from the
        previous restore (no allocation once they exist)."""
        pairs = []
        keep = [self.backup_ssm, self.backup_conv, self.backup_gate_offset]
        spare = [k if k is not None else s for k, s in zip(keep, self._spare)]
        self.backup_ssm = _reuse(spare[0], self.ssm_state)
        self.backup_conv = _reuse(spare[1], self.conv_state)
        pairs += [(self.backup_ssm, self.ssm_state.contiguous()),
                  (self.backup_conv, self.conv_state.contiguous())]
        if self.gate_cumsum_offset is not None:
            self.backup_gate_offset = _reuse(spare[2], self.gate_cumsum_offset)
            pairs.append((self.backup_gate_offset, self.gate_cumsum_offset.contiguous()))
        else:
            self.backup_gate_offset = None
        self._spare = [None, None, None]
        _copy_segments(pairs)

    def restore(self) -> None:
        """RecurrentState::restore (qn:746-757): the backups become the state (O(1)) and are
        taken; gate_cumsum_offset takes the backup's value, None included. The replaced
        tensors are kept for the next checkpoint."""
        if self.backup_ssm is not None:
            self._spare[0], self.ssm_state, self.backup_ssm = self.ssm_state, self.backup_ssm, None
        if self.backup_conv is not None:
            self._spare[1], self.conv_state, self.backup_conv = self.conv_state, self.backup_conv, None
        self._spare[2] = self.gate_cumsum_offset
        self.gate_cumsum_offset, self.backup_gate_offset = self.backup_gate_offset, None


class LinearAttentionState:
    """Recurrent state of one Gated-DeltaNet layer and its per-token step
    (GatedDeltaNet::delta_net_autoregressive, qwen3_next.rs:3392-3470). scale is
    1/sqrt(head_v_dim) (qn:3012-3013), eps the layer's rms_norm_eps; conv_dim and
    conv_kernel size the conv_state created with a first state (qn:3455-3460)."""

    def __init__(self, scale: float = 128 ** -0.5, eps: float = 1e-6, conv_dim: int = 8192,
                 conv_kernel: int = 4):
        self.recurrent_state: Optional[RecurrentState] = None
        self.scale, self.eps = scale, eps
        self.conv_dim, self.conv_kernel = conv_dim, conv_kernel

    def clear_state(self) -> None:
        self.recurrent_state = None

    def checkpoint_state(self) -> None:
        """GatedDeltaNet::checkpoint_state (qn:4011-4019): no state, nothing to save."""
        if self.recurrent_state is not None:
            self.recurrent_state.checkpoint()

    def restore_state(self) -> None:
        """GatedDeltaNet::restore_state (qn:4021-4030)."""
        if self.recurrent_state is not None:
            self.recurrent_state.restore()

    def restore_to_intermediate_state(self, index: int) -> bool:
        """GatedDeltaNet::restore_to_intermediate_state (qn:4046-4054). The per-position
        states come from the chunked verification forward, which is not part of this
        library, so none are held: False, as the reference returns without them."""
        return False

    def delta_net_autoregressive(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                 gate: torch.Tensor, beta: torch.Tensor) -> torch.Tensor:
        """One token. q, k: [b, 1, heads, dk] (repeated to the value heads), v: [b, 1,
        heads, dv], gate (log decay) and beta (pre-sigmoid): [b, 1, heads]. Returns
        [b, 1, heads, dv]. The state [b, heads, dv, dk] is updated in place on the device
        (pkv_deltanet_step); a missing state starts at zero, and gate_cumsum_offset
        accumulates gate (qn:3444-3466)."""
        b, l, H, dk = q.shape
        dv = v.shape[-1]
        if l != 1 or k.shape != q.shape or v.shape[:3] != (b, 1, H):
            raise KvCacheError("delta_net_autoregressive expects one token: q, k [b,1,h,d], v [b,1,h,dv]")
        if dk != dv:
            raise KvCacheError(f"delta_net_autoregressive expects matching head dims ({dk} vs {dv})")
        qq, kk, vv = _f32(q, "q"), _f32(k, "k"), _f32(v, "v")
        g, bt = _f32(gate, "gate"), _f32(beta, "beta")
        rs = self.recurrent_state
        if rs is None:
            rs = RecurrentState(torch.zeros((b, H, dv, dv), dtype=torch.float32, device=q.device),
                                torch.zeros((b, self.conv_dim, self.conv_kernel - 1),
                                            dtype=torch.float32, device=q.device))
            self.recurrent_state = rs
        if rs.gate_cumsum_offset is None:
            rs.gate_cumsum_offset = torch.zeros((b, H), dtype=torch.float32, device=q.device)
        if tuple(rs.ssm_state.shape) != (b, H, dv, dv) or not rs.ssm_state.is_contiguous():
            raise KvCacheError("ssm_state must be a contiguous [b, heads, dv, dk] tensor")
        out = torch.empty_like(vv)
        _call(lib().pkv_deltanet_step(_ptr(qq), _ptr(kk), _ptr(vv), _ptr(g), _ptr(bt),
                                      _ptr(rs.ssm_state), _ptr(rs.gate_cumsum_offset), _ptr(out),
                                      b, H, dv, self.scale, self.eps,
                                      torch.cuda.current_stream().cuda_stream))
        return out


# ------------------------------------------------------------------ PrefixCache
@dataclass
class PrefixCacheEntry:
    """FullAttention / LinearAttention / Empty (qwen3_next.rs:834-854). The payload lives in
    the native prefix object; seq_len (FullAttention) and the state shapes
    (LinearAttention) are kept here."""
    kind: str
    seq_len: int = 0
    shapes: Optional[tuple] = None


@dataclass
class PrefixCache:
    prefix_tokens: List[int]
    layer_caches: List[PrefixCacheEntry] = field(default_factory=list)
    _native: Optional[ctypes.c_void_p] = None

    def __del__(self):
        if self._native is not None and self._native.value:
            self._free(self._native)
            self._native = None

    def to_bytes(self) -> bytes:
        """Host spill: the native blob (pkv_prefix_serialize: tokens, per-layer descriptors,
        packed K/V rows and DeltaNet states as saved), then a JSON trailer with the
        Python-side state shapes and its u64 length."""
        n = lib().pkv_prefix_serialized_size(self._native)
        host = torch.empty(n, dtype=torch.uint8, pin_memory=True)
        _call(lib().pkv_prefix_serialize(self._native, ctypes.c_void_p(host.data_ptr()), n,
                                         ctypes.c_void_p(_stream())))
        meta = json.dumps([[e.kind, e.seq_len, e.shapes] for e in self.layer_caches]).encode()
        return host.numpy().tobytes() + meta + struct.pack("<Q", len(meta))

    @classmethod
    def from_bytes(cls, blob: bytes) -> "PrefixCache":
        """Reload a to_bytes() image into device memory (pkv_prefix_deserialize checks the
        blob's lengths before it allocates)."""
        if len(blob) < 8:
            raise KvCacheError("prefix blob truncated")
        (m,) = struct.unpack("<Q", blob[-8:])
        if m > len(blob) - 8:
            raise KvCacheError("prefix blob truncated")
        native, meta = blob[:len(blob) - 8 - m], json.loads(blob[len(blob) - 8 - m:-8].decode())
        host = torch.frombuffer(bytearray(native), dtype=torch.uint8).pin_memory()
        p = ctypes.c_void_p()
        _call(lib().pkv_prefix_deserialize(ctypes.c_void_p(host.data_ptr()), len(native),
                                           ctypes.byref(p), ctypes.c_void_p(_stream())))
        try:
            entries = cls._check_trailer(p, meta)
        except Exception:
            lib().pkv_prefix_free(p)
            raise
        toks = ctypes.POINTER(ctypes.c_uint32)()
        nt = ctypes.c_size_t()
        _call(lib().pkv_prefix_tokens(p, ctypes.byref(toks), ctypes.byref(nt)))
        pc = cls([toks[i] for i in range(nt.value)], entries, p)
        pc._free = lib().pkv_prefix_free
        return pc

    @staticmethod
    def _check_trailer(p, meta) -> List["PrefixCacheEntry"]:
        """The JSON trailer must describe the native blob exactly: same layer count, kinds,
        FullAttention lengths and LinearAttention element counts (restore sizes its state
        tensors from these shapes)."""
        kinds = {"Empty": _lib.ENTRY_EMPTY, "FullAttention": _lib.ENTRY_FULL,
                 "LinearAttention": _lib.ENTRY_LINEAR}
        if not isinstance(meta, list) or len(meta) != lib().pkv_prefix_num_layers(p):
            raise KvCacheError("prefix blob: trailer layer count differs from the blob")
        entries = []
        for i, item in enumerate(meta):
            if not isinstance(item, list) or len(item) != 3 or item[0] not in kinds:
                raise KvCacheError(f"prefix blob: bad trailer entry {i}")
            kind, n_, sh = item
            if lib().pkv_prefix_entry_kind(p, i) != kinds[kind]:
                raise KvCacheError(f"prefix blob: trailer kind of layer {i} differs from the blob")
            shapes = None
            if kind == "FullAttention":
                if not isinstance(n_, int) or n_ != lib().pkv_prefix_full_len(p, i):
                    raise KvCacheError(f"prefix blob: trailer length of layer {i} differs")
            elif kind == "LinearAttention":
                ns, nc, ng = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
                _call(lib().pkv_prefix_linear_sizes(p, i, ctypes.byref(ns), ctypes.byref(nc),
                                                    ctypes.byref(ng)))
                try:
                    shapes = tuple(tuple(int(d) for d in x) for x in sh)
                    ok = len(shapes) == 3 and all(d >= 0 for x in shapes for d in x) and \
                        [int(np_prod(x)) for x in shapes] == [ns.value, nc.value, ng.value]
                except (TypeError, ValueError):
                    ok = False
                if not ok:
                    raise KvCacheError(f"prefix blob: trailer state shapes of layer {i} differ")
            entries.append(PrefixCacheEntry(kind, n_ if kind == "FullAttention" else 0, shapes))
        return entries


class ModelKvState:
    """Cache management of ModelWeights restricted to the attention state: a list of
    layers, full attention where (i+1) % interval == 0 (qwen3_next.rs:4574-4583)."""

    def __init__(self, n_layers: int, full_attention_interval: int, num_heads: int,
                 num_kv_heads: int, head_dim: int, max_seq_len: int,
                 quant: KvCacheQuantization = KvCacheQuantization.Q4K):
        self.layers = []
        for i in range(n_layers):
            if (i + 1) % full_attention_interval == 0:
                self.layers.append(FullAttentionKv(num_heads, num_kv_heads, head_dim, max_seq_len, quant))
            else:
                self.layers.append(LinearAttentionState())

    def full_layers(self) -> List[FullAttentionKv]:
        return [l for l in self.layers if isinstance(l, FullAttentionKv)]

    def clear_kv_cache(self) -> None:
        for l in self.layers:
            if isinstance(l, FullAttentionKv):
                l.clear_kv_cache()
            else:
                l.clear_state()

    clear_cache = clear_kv_cache

    def truncate_cache(self, new_len: int) -> None:
        """Full layers truncate, linear layers clear (qwen3_next.rs:4301-4306)."""
        for l in self.layers:
            if isinstance(l, FullAttentionKv):
                l.truncate_kv_cache(new_len)
            else:
                l.clear_state()

    def cache_seq_len(self) -> int:
        for l in self.layers:
            if isinstance(l, FullAttentionKv):
                return l.cache_seq_len()
        return 0

    def checkpoint_cache(self) -> List[LayerCheckpoint]:
        """ModelWeights::checkpoint_cache (qn:5479-5488, per layer :4311-4322)."""
        out = []
        for l in self.layers:
            if isinstance(l, FullAttentionKv):
                out.append(l.checkpoint())
            else:
                l.checkpoint_state()
                out.append(LayerCheckpoint("LinearAttention"))
        return out

    def restore_cache(self, checkpoints: Sequence[LayerCheckpoint]) -> None:
        """ModelWeights::restore_cache (qn:5490-5501, per layer :4326-4341); a checkpoint of
        the other layer kind is ignored, as the reference's match does."""
        for l, cp in zip(self.layers, checkpoints):
            if isinstance(l, FullAttentionKv) and cp.kind == "FullAttention":
                l.restore(cp.seq_len)
            elif isinstance(l, LinearAttentionState) and cp.kind == "LinearAttention":
                l.restore_state()

    def restore_to_intermediate_state(self, index: int, offset: int) -> None:
        """ModelWeights::restore_to_intermediate_state (qn:5377-5381, per layer :4365-4375):
        full layers truncate to offset + index + 1."""
        for l in self.layers:
            if isinstance(l, FullAttentionKv):
                l.truncate_kv_cache(offset + index + 1)
            else:
                l.restore_to_intermediate_state(index)

    def save_prefix_cache(self, prefix_tokens: Sequence[int]) -> PrefixCache:
        toks = (ctypes.c_uint32 * max(len(prefix_tokens), 1))(*prefix_tokens)
        p = ctypes.c_void_p()
        _call(lib().pkv_prefix_create(toks, len(prefix_tokens), len(self.layers), ctypes.byref(p)))
        pc = PrefixCache(list(prefix_tokens), [], p)
        pc._free = lib().pkv_prefix_free  # held for __del__ at interpreter shutdown
        s = ctypes.c_void_p(_stream())
        for i, l in enumerate(self.layers):
            if isinstance(l, FullAttentionKv):
                c = l.quantized_cache
                if c is not None and c.seq_len > 0:
                    _call(lib().pkv_prefix_save_full(p, i, c.handle))
                    pc.layer_caches.append(PrefixCacheEntry("FullAttention", c.seq_len))
                else:
                    pc.layer_caches.append(PrefixCacheEntry("Empty"))
            else:
                rs = l.recurrent_state
                if rs is None:
                    pc.layer_caches.append(PrefixCacheEntry("Empty"))
                    continue
                ssm, conv = rs.ssm_state.contiguous(), rs.conv_state.contiguous()
                gate = rs.gate_cumsum_offset
                gshape = (ssm.shape[0], ssm.shape[1])
                _call(lib().pkv_prefix_save_linear(
                    p, i, _ptr(ssm), ssm.numel(), _ptr(conv), conv.numel(),
                    _ptr(gate.contiguous()) if gate is not None else None,
                    gshape[0] * gshape[1], s))
                pc.layer_caches.append(PrefixCacheEntry(
                    "LinearAttention", shapes=(tuple(ssm.shape), tuple(conv.shape), gshape)))
        return pc

    def restore_prefix_cache(self, cache: PrefixCache, requantize: bool = False) -> int:
        """All layers restore in one batched copy launch; requantize=True reproduces the
        reference's clear()+append(dequantized) bytes instead of the exact snapshot."""
        n = len(self.layers)
        p = cache._native
        if len(cache.layer_caches) != n or lib().pkv_prefix_num_layers(p) != n:
            raise PrefixLayerMismatch(
                f"Prefix cache layer count mismatch: {len(cache.layer_caches)} vs {n}")
        targets = (_lib.LayerTarget * n)()
        valid = (ctypes.c_int * n)()
        restored = {}
        for i, l in enumerate(self.layers):
            kind = lib().pkv_prefix_entry_kind(p, i)
            if isinstance(l, FullAttentionKv):
                if kind == _lib.ENTRY_FULL and l.quantized_cache is None:
                    l._ensure(1)  # lazily created with max_seq_len (qwen3_next.rs:2830-2840)
                if l.quantized_cache is not None:
                    targets[i].cache = l.quantized_cache.handle.value
                continue
            if kind == _lib.ENTRY_LINEAR:
                ss, cs, gs = cache.layer_caches[i].shapes
                t = tuple(torch.empty(sh, dtype=torch.float32, device="cuda") for sh in (ss, cs, gs))
                restored[i] = t
                targets[i].ssm, targets[i].conv, targets[i].gate_offset = (x.data_ptr() for x in t)
                targets[i].ssm_cap, targets[i].conv_cap, targets[i].gate_cap = (x.numel() for x in t)
            targets[i].state_valid = ctypes.cast(ctypes.addressof(valid) + 4 * i,
                                                 ctypes.POINTER(ctypes.c_int))
        ntok = ctypes.c_size_t()
        mode = _lib.RESTORE_REQUANTIZE if requantize else _lib.RESTORE_BYTES
        _call(lib().pkv_prefix_restore(p, targets, n, mode, ctypes.byref(ntok),
                                       ctypes.c_void_p(_stream())))
        for i, l in enumerate(self.layers):
            if isinstance(l, LinearAttentionState):
                if valid[i] and i in restored:
                    l.recurrent_state = RecurrentState(*restored[i])
                else:
                    l.clear_state()  # Empty or wrong kind (qwen3_next.rs:4121-4130)
        return ntok.value
