"""GGUF weight blocks for the output-projection tests, built element by element from the
published block layouts (ggml-common.h block_q5_K / block_q6_K / block_q4_K / block_q8_0),
independently of the oracle's decoders: a packer takes per-element codes and per-sub-block
scales and places every bit where the format says it lives.

Layouts (bytes):
  Q8_0  34: f16 d, 32 int8 codes; y = d * q
  Q4K  144: f16 d, f16 dmin, 12 B 6-bit (scale, min) codes, 128 B nibbles
  Q5K  176: f16 d, f16 dmin, 12 B 6-bit (scale, min) codes, 32 B high bits, 128 B nibbles
  Q6K  210: 128 B low nibbles, 64 B high bit pairs, 16 int8 scales, f16 d
"""
import numpy as np

W_Q8_0, W_Q4K, W_Q5K, W_Q6K = 8, 12, 13, 14
W_BLOCK = {W_Q8_0: 32, W_Q4K: 256, W_Q5K: 256, W_Q6K: 256}
W_BLOCK_BYTES = {W_Q8_0: 34, W_Q4K: 144, W_Q5K: 176, W_Q6K: 210}
NAMES = {W_Q8_0: "q8_0", W_Q4K: "q4k", W_Q5K: "q5k", W_Q6K: "q6k"}


def f16_bytes(v):
    return np.array([v], dtype=np.float16).view(np.uint8)


def pack_scale_min_k4(ls, lm):
    """The 12-byte 6-bit (scale, min) packing shared by Q4K and Q5K: sub-blocks 0-3 keep
    their 6 bits in bytes j and j + 4; sub-blocks 4-7 keep the low 4 bits in byte j + 4
    (scale low nibble, min high nibble) and the top 2 bits in bits 6-7 of bytes j - 4
    (scale) and j (min)."""
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


def pack_q4k(d, dmin, ls, lm, codes):
    """codes: 256 values 0..15; element 64 c + l is the low nibble of byte 32 c + l,
    element 64 c + 32 + l its high nibble; sub-block j = element // 32."""
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2], blk[2:4] = f16_bytes(d), f16_bytes(dmin)
    blk[4:16] = pack_scale_min_k4(ls, lm)
    for e in range(256):
        c, r = divmod(e, 64)
        hi, l = divmod(r, 32)
        blk[16 + 32 * c + l] |= (int(codes[e]) & 15) << (4 * hi)
    return blk


def pack_q5k(d, dmin, ls, lm, codes):
    """codes: 256 values 0..31. The low 4 bits sit as in Q4K (bytes 48..175); bit 4 of
    element e = 32 j + l (sub-block j) is bit j of high-bit byte l (bytes 16..47)."""
    blk = np.zeros(176, dtype=np.uint8)
    blk[0:2], blk[2:4] = f16_bytes(d), f16_bytes(dmin)
    blk[4:16] = pack_scale_min_k4(ls, lm)
    for e in range(256):
        j, l = divmod(e, 32)
        c, hi = divmod(j, 2)
        blk[48 + 32 * c + l] |= (int(codes[e]) & 15) << (4 * hi)
        blk[16 + l] |= ((int(codes[e]) >> 4) & 1) << j
    return blk


def pack_q6k(d, scales, codes):
    """codes: 256 values 0..63 (the stored unsigned code; the value is code - 32), scales:
    16 int8, element e scaled by scales[e // 16]. Element e = 128 h + 32 g + l: low 4 bits
    in byte 64 h + l + 32 (g % 2) of the low-nibble array (low nibble for g < 2, high
    nibble for g >= 2), bits 4-5 in bits 2 g, 2 g + 1 of byte 32 h + l of the high-bit
    array (bytes 128..191); scales at bytes 192..207, d at 208..209."""
    blk = np.zeros(210, dtype=np.uint8)
    for e in range(256):
        h, r = divmod(e, 128)
        g, l = divmod(r, 32)
        blk[64 * h + l + 32 * (g % 2)] |= (int(codes[e]) & 15) << (4 * (g // 2))
        blk[128 + 32 * h + l] |= ((int(codes[e]) >> 4) & 3) << (2 * g)
    blk[192:208] = np.asarray(scales, dtype=np.int8).view(np.uint8)
    blk[208:210] = f16_bytes(d)
    return blk


def pack_q8_0(d, codes):
    blk = np.zeros(34, dtype=np.uint8)
    blk[0:2] = f16_bytes(d)
    blk[2:34] = np.asarray(codes, dtype=np.int8).view(np.uint8)
    return blk


def random_weight_bytes(rng, w_type, out_dim, in_dim, d_scale=2e-3):
    """out_dim rows of in_dim elements in GGUF type w_type: random codes and scale codes,
    and finite f16 (d, dmin) of about d_scale, so that dot products over a few thousand
    inputs stay O(1). Vectorised (the per-element packers above are for small cases)."""
    nb = out_dim * in_dim // W_BLOCK[w_type]
    blk = rng.integers(0, 256, (nb, W_BLOCK_BYTES[w_type]), dtype=np.uint8)
    d = (np.abs(rng.standard_normal(nb)) * d_scale + d_scale / 8).astype(np.float16)
    if w_type == W_Q6K:
        blk[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    else:
        blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    if w_type in (W_Q4K, W_Q5K):
        dmin = (np.abs(rng.standard_normal(nb)) * d_scale).astype(np.float16)
        blk[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    return np.ascontiguousarray(blk.reshape(-1))
