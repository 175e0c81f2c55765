"""pkv_flash_attn_noalloc: the flash-attention entry point for callers that cannot
allocate (graph capture, serving loops). Through the C ABI it must give the same output
as pkv_flash_attn on the same inputs, on calls in a row of different sizes (the static
scratch keeps the previous call's contents), refuse a plan beyond its scratch before
enqueueing anything, and leave the device's free memory unchanged."""
import ctypes
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


@pytest.fixture(scope="module")
def ready(pk):
    """The first call on a device is the set-up: HIP places the library's static scratch
    on the device when its address is first looked up. Later calls must allocate nothing."""
    c = make_cache(pk, pk.KvCacheQuantization.Q4K, 1, 64, 1)
    q = torch.randn((1, 1, 16, 256), device="cuda")
    out = torch.empty_like(q)
    assert call("pkv_flash_attn_noalloc", pk.KvCacheQuantization.Q4K, c, q, 1, 63, True, out) == 0
    torch.cuda.synchronize()
    return pk


def free_device_bytes():
    return torch.cuda.mem_get_info()[0]  # hipMemGetInfo


def make_cache(pk, quant, B, S, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    c = pk.PreallocatedQuantizedKvCache(B, 2, S, 256, quant)
    c.append_quantized(torch.randn((B, 2, S, 256), device="cuda", generator=g),
                       torch.randn((B, 2, S, 256), device="cuda", generator=g))
    return c


def call(fn_name, quant, c, q, seq_q, q_offset, causal, out):
    from paramecia_amd._lib import lib
    kp, vp, _, st = c.get_kv_storage()
    strides = (ctypes.c_int64 * 3)(*st[:3])
    B, _, H, D = q.shape
    rc = getattr(lib(), fn_name)(int(quant), ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(kp),
                                 ctypes.c_void_p(vp), strides, 1.0 / 16, B, H, 2, D, seq_q,
                                 c.seq_len, q_offset, int(causal), ctypes.c_void_p(out.data_ptr()),
                                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    return rc


def compare(pk, quant, B, S, seq_q, seed):
    c = make_cache(pk, quant, B, S, seed)
    q = torch.randn((B, seq_q, 16, 256), device="cuda",
                    generator=torch.Generator(device="cuda").manual_seed(seed + 1))
    ref = torch.empty_like(q)
    got = torch.full_like(q, float("nan"))
    assert call("pkv_flash_attn", quant, c, q, seq_q, S - seq_q, True, ref) == 0
    torch.cuda.synchronize()
    before = free_device_bytes()
    assert call("pkv_flash_attn_noalloc", quant, c, q, seq_q, S - seq_q, True, got) == 0
    torch.cuda.synchronize()
    assert free_device_bytes() == before, "the no-alloc call changed the device's free memory"
    a, b = got.cpu().numpy(), ref.cpu().numpy()
    assert np.array_equal(a, b), f"max |diff| {np.abs(a - b).max():.3e}"


def test_noalloc_matches_flash_attn_calls_in_a_row(ready):
    pk = ready
    Q = pk.KvCacheQuantization
    say("no-alloc: Q4K decode, 131073 keys (4.7 MB of partials)")
    compare(pk, Q.Q4K, 1, 131073, 1, 40)
    say("no-alloc: Q4K decode, batch 2, 5000 keys (smaller, after the larger call)")
    compare(pk, Q.Q4K, 2, 5000, 1, 41)
    say("no-alloc: Q8_0 decode, 4097 keys")
    compare(pk, Q.Q8_0, 1, 4097, 1, 42)
    say("no-alloc: F16 generic path, 3 queries over 700 keys")
    compare(pk, Q.F16, 1, 700, 3, 43)


def test_noalloc_refuses_plan_beyond_scratch(ready):
    pk = ready
    from paramecia_amd._lib import ERR_ARG, lib
    say("no-alloc: a Q4K prefill chunk needing more than the scratch is refused")
    c = make_cache(pk, pk.KvCacheQuantization.Q4K, 1, 16896, 44)
    q = torch.randn((1, 512, 16, 256), device="cuda")
    out = torch.full_like(q, float("nan"))
    torch.cuda.synchronize()
    assert call("pkv_flash_attn_noalloc", pk.KvCacheQuantization.Q4K, c, q, 512, 16896 - 512,
                True, out) == ERR_ARG
    assert b"scratch" in lib().pkv_last_error()
    torch.cuda.synchronize()
    assert torch.isnan(out).all(), "a refused call wrote its output"
