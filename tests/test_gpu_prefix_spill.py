"""PrefixCache host spill (pkv_prefix_serialize / pkv_prefix_deserialize; PrefixCache.to_bytes
and from_bytes): a prefix of full-attention K/V rows and Gated-DeltaNet states goes to host
memory and back, and the restore from the reloaded prefix gives the saved bytes exactly.
The reference keeps prefixes in device memory only (qwen3_next.rs:856-864); blobs that are
truncated or altered are refused before anything is allocated."""
import ctypes
import struct
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def pk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import paramecia_amd
    paramecia_amd.lib()
    return paramecia_amd


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def model_with_state(pk, quant):
    m = pk.ModelKvState(8, 4, 16, 2, 256, 64, quant)
    g = torch.Generator(device="cuda").manual_seed(5)
    for l in m.layers:
        if isinstance(l, pk.FullAttentionKv):
            k = torch.randn((1, 2, 20, 256), device="cuda", generator=g)
            v = torch.randn((1, 2, 20, 256), device="cuda", generator=g)
            l._ensure(1).append_quantized(k, v)
        else:
            l.recurrent_state = pk.RecurrentState(
                torch.randn((1, 32, 128, 128), device="cuda", generator=g) * 0.02,
                torch.randn((1, 8192, 3), device="cuda", generator=g),
                torch.randn((1, 32), device="cuda", generator=g))
    return m


def snapshot(pk, m):
    out = []
    for l in m.layers:
        if isinstance(l, pk.FullAttentionKv):
            out.append(tuple(host(x) for x in l.quantized_cache.raw_bytes()))
        else:
            rs = l.recurrent_state
            out.append((host(rs.ssm_state), host(rs.conv_state), host(rs.gate_cumsum_offset)))
    return out


@pytest.mark.parametrize("quant", ["Q4K", "Q8_0"])
def test_spill_and_reload_restores_exact_bytes(pk, quant):
    say(f"prefix spill round trip {quant}")
    m = model_with_state(pk, getattr(pk.KvCacheQuantization, quant))
    before = snapshot(pk, m)
    pc = m.save_prefix_cache(list(range(20)))
    blob = pc.to_bytes()
    del pc
    pc2 = pk.PrefixCache.from_bytes(blob)
    assert pc2.prefix_tokens == list(range(20))
    # change every layer, then restore from the reloaded prefix
    for l in m.layers:
        if isinstance(l, pk.FullAttentionKv):
            l.quantized_cache.append_quantized(torch.randn((1, 2, 5, 256), device="cuda"),
                                               torch.randn((1, 2, 5, 256), device="cuda"))
        else:
            l.clear_state()
    assert m.restore_prefix_cache(pc2) == 20
    after = snapshot(pk, m)
    for a, b in zip(before, after):
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)


def test_refuses_bad_blobs(pk):
    from paramecia_amd._lib import lib, ERR_ARG
    say("prefix spill: bad blobs")
    m = model_with_state(pk, pk.KvCacheQuantization.Q4K)
    pc = m.save_prefix_cache([1, 2, 3])
    blob = pc.to_bytes()
    (meta,) = struct.unpack("<Q", blob[-8:])
    native = bytearray(blob[:len(blob) - 8 - meta])

    def load(b):
        buf = (ctypes.c_uint8 * len(b)).from_buffer(b)
        p = ctypes.c_void_p()
        rc = lib().pkv_prefix_deserialize(ctypes.addressof(buf), len(b), ctypes.byref(p), None)
        if rc == 0:
            lib().pkv_prefix_free(p)
        return rc

    assert load(bytearray(native)) == 0
    assert load(bytearray(native[:-1])) == ERR_ARG           # truncated payload
    assert load(bytearray(native[:16])) == ERR_ARG           # truncated header
    bad = bytearray(native)
    bad[0] ^= 0xFF                                           # magic
    assert load(bad) == ERR_ARG
    table = 32 + 16                    # 32-byte header, 3 tokens padded to 16 bytes
    entry = 64                         # six int32 then five u64 per layer
    bad = bytearray(native)            # layer 0 (linear): n_ssm beyond the blob
    bad[table + 40:table + 48] = struct.pack("<Q", 1 << 40)
    assert load(bad) == ERR_ARG
    bad = bytearray(native)            # layer 3 (full attention): bytes per row
    bad[table + 3 * entry + 24:table + 3 * entry + 32] = struct.pack("<Q", 1 << 40)
    assert load(bad) == ERR_ARG
    bad = bytearray(native)            # layer 3: a length that overflows the product
    bad[table + 3 * entry + 32:table + 3 * entry + 40] = struct.pack("<Q", (1 << 63) + 7)
    assert load(bad) == ERR_ARG
    with pytest.raises(Exception):
        pk.PrefixCache.from_bytes(blob[:20])


def _retrailer(blob, fn):
    """The blob with its JSON trailer rewritten by fn (the native part unchanged)."""
    import json
    (m,) = struct.unpack("<Q", blob[-8:])
    native, meta = blob[:len(blob) - 8 - m], json.loads(blob[len(blob) - 8 - m:-8].decode())
    meta = fn(meta)
    t = json.dumps(meta).encode()
    return native + t + struct.pack("<Q", len(t))


def test_refuses_trailer_that_disagrees_with_blob(pk):
    """The Python trailer sizes the restored state tensors, so it must match the native
    blob: smaller state shapes, a wrong kind, a wrong length or a missing layer are
    refused before any restore."""
    say("prefix spill: trailer checks")
    m = model_with_state(pk, pk.KvCacheQuantization.Q4K)
    blob = m.save_prefix_cache([7, 8]).to_bytes()
    pk.PrefixCache.from_bytes(blob)  # unaltered: accepted

    def smaller_state(meta):
        meta[0][2][0] = [1, 32, 64, 128]       # layer 0 (linear): half the ssm rows
        return meta

    def wrong_kind(meta):
        meta[3] = ["Empty", 0, None]            # layer 3 is full attention in the blob
        return meta

    def wrong_len(meta):
        meta[3][1] = 19
        return meta

    def linear_as_empty(meta):
        meta[1] = ["Empty", 0, None]
        return meta

    for fn in (smaller_state, wrong_kind, wrong_len, linear_as_empty, lambda m_: m_[:-1]):
        with pytest.raises(pk.KvCacheError):
            pk.PrefixCache.from_bytes(_retrailer(blob, fn))


def test_restore_refuses_small_state_targets(pk):
    """pkv_prefix_restore checks each state target's capacity against the saved counts
    (PKV_ERR_LAYOUT) before it writes anything."""
    from paramecia_amd._lib import lib, LayerTarget, ERR_LAYOUT
    say("prefix restore: state target capacities")
    m = model_with_state(pk, pk.KvCacheQuantization.Q4K)
    pc = m.save_prefix_cache([1])
    n = len(m.layers)
    targets = (LayerTarget * n)()
    keep = []
    for i, l in enumerate(m.layers):
        if isinstance(l, pk.FullAttentionKv):
            targets[i].cache = l.quantized_cache.handle.value
        else:
            rs = l.recurrent_state
            t = (torch.empty_like(rs.ssm_state), torch.empty_like(rs.conv_state),
                 torch.empty_like(rs.gate_cumsum_offset))
            keep.append(t)
            targets[i].ssm, targets[i].conv, targets[i].gate_offset = (x.data_ptr() for x in t)
            targets[i].ssm_cap, targets[i].conv_cap, targets[i].gate_cap = (x.numel() for x in t)
    targets[2].conv_cap -= 1
    lens = [l.quantized_cache.seq_len for l in m.full_layers()]
    rc = lib().pkv_prefix_restore(pc._native, targets, n, 0, None, None)
    assert rc == ERR_LAYOUT, lib().pkv_last_error()
    assert [l.quantized_cache.seq_len for l in m.full_layers()] == lens
    targets[2].conv_cap += 1
    assert lib().pkv_prefix_restore(pc._native, targets, n, 0, None, None) == 0
    torch.cuda.synchronize()
