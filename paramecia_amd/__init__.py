"""paramecia_amd — MI355X-native quantized KV-cache path of paramecia-model.

The kernels and the C ABI live in libpkv.so (csrc/, include/pkv.h); this package is the
host-side mirror of the reference's Rust API used by tests and the benchmark.
"""
from ._lib import PkvError, lib  # noqa: F401
from .kv_cache import (  # noqa: F401
    EmptyCacheError, FullAttentionKv, KvCacheError, KvCacheOffsetMismatch, KvCacheOverflow,
    KvCacheQuantization, LayerCheckpoint, LinearAttentionState, ModelKvState, PagedKvPool,
    PagedSequence, PreallocatedQuantizedKvCache,
    PrefixCache, PrefixCacheEntry, PrefixLayerMismatch, QkPrep, RecurrentState, RotaryEmbedding,
    append_attend_batched, fill_normal, flash_attn, gated_o_proj, scale_channels,
    WTYPE_Q4K, WTYPE_Q5K, WTYPE_Q6K, WTYPE_Q8_0,
)
