"""CPU checks of the PrefixCache blob parser (pkv_prefix_deserialize): every malformed blob
is refused with PKV_ERR_ARG before any HIP call or allocation, so these run without a GPU.
Blob layout: a 32-byte header (magic "PKVP", version 1, n_tokens, n_layers, total bytes),
the tokens (u32, padded to 8 bytes), 64-byte layer descriptors (kind, quant, batch,
heads, head_dim, pad as i32; bpr, len, n_ssm, n_conv, n_gate as u64), then payloads."""
import ctypes
import struct

import pytest

from paramecia_amd import _lib

MAGIC, VERSION = 0x50564B50, 1
FULL, LINEAR = 1, 2
Q4K = 4


def header(n_tokens, n_layers, total):
    return struct.pack("<IIQQQ", MAGIC, VERSION, n_tokens, n_layers, total)


def entry(kind, quant=0, batch=0, heads=0, head_dim=0, bpr=0, length=0, n_ssm=0, n_conv=0, n_gate=0):
    return struct.pack("<6i5Q", kind, quant, batch, heads, head_dim, 0, bpr, length, n_ssm, n_conv, n_gate)


def load(blob):
    buf = (ctypes.c_uint8 * max(len(blob), 1)).from_buffer_copy(blob + b"\0")
    p = ctypes.c_void_p()
    return _lib.lib().pkv_prefix_deserialize(ctypes.addressof(buf), len(blob), ctypes.byref(p), None)


def full_blob(bpr=144, length=2, batch=1, heads=2, payload=None):
    body = struct.pack("<II", 7, 8) + entry(FULL, Q4K, batch, heads, 256, bpr, length)
    nbytes = length * batch * heads * bpr
    pay = payload if payload is not None else bytes(2 * ((nbytes + 7) // 8 * 8))
    total = 32 + len(body) + len(pay)
    return header(2, 1, total) + body + pay


@pytest.mark.parametrize("case", ["short", "magic", "version", "total", "layers", "bpr",
                                  "bpr_huge", "len_overflow", "payload_short", "payload_long",
                                  "kind", "linear_huge"])
def test_malformed_blob_is_refused(case):
    good = full_blob()
    make = {
        "short": lambda: good[:31],
        "magic": lambda: b"XKVP" + good[4:],
        "version": lambda: good[:4] + struct.pack("<I", 2) + good[8:],
        "total": lambda: good[:24] + struct.pack("<Q", len(good) + 8) + good[32:],
        "layers": lambda: good[:16] + struct.pack("<Q", 1 << 40) + good[24:],
        "bpr": lambda: full_blob(bpr=145),
        "bpr_huge": lambda: full_blob(bpr=1 << 40, payload=b""),
        "len_overflow": lambda: full_blob(length=(1 << 63) + 3, payload=b""),
        "payload_short": lambda: full_blob(payload=bytes(8)),
        "payload_long": lambda: full_blob(payload=bytes(2 * 576 + 64)),
        "kind": lambda: header(0, 1, 32 + 64) + entry(9),
        "linear_huge": lambda: header(0, 1, 32 + 64) + entry(LINEAR, n_ssm=1 << 50),
    }
    blob = make[case]()
    assert load(blob) == _lib.ERR_ARG
    assert _lib.lib().pkv_last_error()
