"""Workload shapes of the benchmark configurations and the seeded stream ids of their
synthetic tensors, shared by bench.py and the tests so both draw identical data.

Qwen3-Next-80B-A3B full-attention layer: 16 query heads, 2 KV heads, head_dim 256,
softmax scale 1/16; 48 layers of which every fourth is full attention (12).
"""
from __future__ import annotations

from dataclasses import dataclass

NUM_HEADS = 16
NUM_KV_HEADS = 2
HEAD_DIM = 256
SCALE = 1.0 / 16.0
N_ROT = 64                                   # rope.dimension_count (25% of head_dim)
ROPE_THETA = 1.0e7                           # rope.freq_base
RMS_EPS = 1e-6                               # attention.layer_norm_rms_epsilon
HIDDEN = 2048                                # embedding_length (wo: 4096 -> 2048)
N_LAYERS = 48
FULL_INTERVAL = 4
N_FULL = N_LAYERS // FULL_INTERVAL          # 12
N_LINEAR = N_LAYERS - N_FULL                # 36
DN_HEADS, DN_DK, DN_DV = 32, 128, 128        # Gated-DeltaNet value heads and state dims
DN_CONV_DIM, DN_CONV_K = 8192, 4             # conv state [conv_dim, k-1]
SEED = 0x5EED_2026

# tensor codes of the stream id
T_PREFILL_K, T_PREFILL_V, T_Q, T_NEW_K, T_NEW_V = 0, 1, 2, 3, 4
T_SSM, T_CONV, T_GATE, T_SUFFIX_K, T_SUFFIX_V = 5, 6, 7, 8, 9
T_CHUNK_K, T_CHUNK_V, T_CHUNK_Q, T_LENGTHS, T_CHANNELS = 10, 11, 12, 13, 14
T_DN_Q, T_DN_K, T_DN_V, T_DN_GATE, T_DN_BETA = 15, 16, 17, 18, 19
T_WO = 20


def stream_id(config: int, tensor: int, layer: int = 0, seq: int = 0) -> int:
    return (config << 56) | (seq << 40) | (layer << 24) | tensor


@dataclass(frozen=True)
class Config:
    index: int
    quant: str
    cached: int        # tokens already in the cache
    capacity: int
    layers: int
    new_tokens: int    # appended per step (chunk for config 2)


CONFIGS = {
    1: Config(1, "Q8_0", 4096, 4097, 1, 1),
    2: Config(2, "Q4K", 16384, 32768, 1, 512),
    3: Config(3, "Q4K", 131072, 131073, N_FULL, 1),
    4: Config(4, "Q4K", 65536, 131072, N_FULL, 1024),
    5: Config(5, "Q4K", 0, 65537, N_FULL, 1),
}

# config 5: 16 sequences, lengths uniform in [1024, 65536], 2% of head_dim channels x20
C5_SEQS = 16
C5_MIN_LEN, C5_MAX_LEN = 1024, 65536
C5_OUTLIER_CHANNELS = round(0.02 * HEAD_DIM)  # 5
C5_OUTLIER_SCALE = 20.0


def c5_lengths(seed: int = SEED):
    """Seeded cached lengths of config 5 (Philox-free: a fixed LCG over the seed)."""
    x = seed & 0xFFFFFFFF
    out = []
    for _ in range(C5_SEQS):
        x = (1103515245 * x + 12345) & 0x7FFFFFFF
        out.append(C5_MIN_LEN + x % (C5_MAX_LEN - C5_MIN_LEN + 1))
    return out


def c5_channels(seed: int = SEED):
    x = (seed >> 7) & 0xFFFFFFFF
    chans = []
    while len(chans) < C5_OUTLIER_CHANNELS:
        x = (1103515245 * x + 12345) & 0x7FFFFFFF
        c = x % HEAD_DIM
        if c not in chans:
            chans.append(c)
    return sorted(chans)


# GGUF weight types of the output projection (GGML numbering) and their block geometry
W_TYPES = {"q8_0": 8, "q4k": 12, "q5k": 13, "q6k": 14}
W_BLOCK = {8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


def kquant_rows(w_type: int, out_dim: int, in_dim: int, seed: int, d_scale: float = 1e-4):
    """Synthetic GGUF weight bytes: out_dim rows of in_dim inputs of type w_type with
    uniform random codes and scale codes and finite f16 (d, dmin) of about d_scale (so a
    row dotted with N(0, 1) inputs stays O(1)). numpy, seeded; uint8 [out_dim * row bytes]."""
    import numpy as np
    blk, nbytes = W_BLOCK[w_type]
    nb = out_dim * in_dim // blk
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (nb, nbytes), dtype=np.uint8)
    d = (np.abs(rng.standard_normal(nb)) * d_scale + d_scale / 8).astype(np.float16)
    if w_type == 14:
        b[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    else:
        b[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    if w_type in (12, 13):
        dmin = (np.abs(rng.standard_normal(nb)) * d_scale).astype(np.float16)
        b[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    return np.ascontiguousarray(b.reshape(-1))
