"""Speculative-decoding rewind hooks of ModelWeights (qwen3_next.rs:4301-4375, 5466-5501):
truncate_cache, checkpoint_cache / restore_cache and restore_to_intermediate_state, with
the reference's behaviour for quantized caches (a checkpoint reads preallocated_cache,
the F16 / BF16 cache, so a Q8_0 / Q4K cache checkpoints length 0 and is left alone on
restore) and for the Gated-DeltaNet layers (state copied to backups, swapped back)."""
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


def make_model(pk, quant, n_tok=12, seed=3):
    """8 layers, every 4th full attention (2 full, 6 linear), n_tok tokens in the caches
    and one DeltaNet step run on every linear layer."""
    m = pk.ModelKvState(8, 4, 16, 2, 256, 64, quant)
    g = torch.Generator(device="cuda").manual_seed(seed)
    for l in m.layers:
        if isinstance(l, pk.FullAttentionKv):
            l._ensure(1).append_quantized(torch.randn((1, 2, n_tok, 256), device="cuda", generator=g),
                                          torch.randn((1, 2, n_tok, 256), device="cuda", generator=g))
        else:
            step(l, g)
    return m, g


def step(l, g, H=4, d=64):
    q = torch.randn((1, 1, H, d), device="cuda", generator=g)
    k = torch.randn((1, 1, H, d), device="cuda", generator=g)
    v = torch.randn((1, 1, H, d), device="cuda", generator=g)
    gate = -torch.rand((1, 1, H), device="cuda", generator=g)
    beta = torch.randn((1, 1, H), device="cuda", generator=g)
    return l.delta_net_autoregressive(q, k, v, gate, beta)


def states(pk, m):
    out = []
    for l in m.layers:
        if isinstance(l, pk.LinearAttentionState):
            rs = l.recurrent_state
            out.append(None if rs is None else (
                host(rs.ssm_state), host(rs.conv_state),
                None if rs.gate_cumsum_offset is None else host(rs.gate_cumsum_offset)))
    return out


def test_truncate_cache(pk):
    say("rewind: truncate_cache")
    m, _ = make_model(pk, pk.KvCacheQuantization.Q4K)
    assert m.cache_seq_len() == 12
    m.truncate_cache(5)
    assert [l.cache_seq_len() for l in m.full_layers()] == [5, 5]
    # linear layers cannot truncate a recurrent state: they clear it (qn:4301-4306)
    assert all(l.recurrent_state is None for l in m.layers if isinstance(l, pk.LinearAttentionState))
    m.truncate_cache(9)  # longer than the cache: nothing changes
    assert m.cache_seq_len() == 5


@pytest.mark.parametrize("quant", ["Q4K", "Q8_0"])
def test_checkpoint_quantized_cache_is_not_rewound(pk, quant):
    """The reference's quirk: checkpoint_cache reads preallocated_cache (F16 / BF16 only),
    so a quantized layer checkpoints seq_len 0 and restore_cache leaves it as it is."""
    say(f"rewind: checkpoint / restore, {quant}")
    m, g = make_model(pk, getattr(pk.KvCacheQuantization, quant))
    cps = m.checkpoint_cache()
    assert [c.kind for c in cps] == ["LinearAttention"] * 3 + ["FullAttention"] + \
        ["LinearAttention"] * 3 + ["FullAttention"]
    assert [c.seq_len for c in cps if c.kind == "FullAttention"] == [0, 0]
    for l in m.full_layers():
        l.quantized_cache.append_quantized(torch.randn((1, 2, 3, 256), device="cuda"),
                                           torch.randn((1, 2, 3, 256), device="cuda"))
    m.restore_cache(cps)
    assert [l.cache_seq_len() for l in m.full_layers()] == [15, 15]


@pytest.mark.parametrize("quant", ["F16", "BF16"])
def test_checkpoint_float_cache_rewinds(pk, quant):
    say(f"rewind: checkpoint / restore, {quant}")
    m, _ = make_model(pk, getattr(pk.KvCacheQuantization, quant))
    before = [tuple(host(x) for x in l.quantized_cache.raw_bytes()) for l in m.full_layers()]
    cps = m.checkpoint_cache()
    assert [c.seq_len for c in cps if c.kind == "FullAttention"] == [12, 12]
    for l in m.full_layers():
        l.quantized_cache.append_quantized(torch.randn((1, 2, 4, 256), device="cuda"),
                                           torch.randn((1, 2, 4, 256), device="cuda"))
    m.restore_cache(cps)
    assert [l.cache_seq_len() for l in m.full_layers()] == [12, 12]
    after = [tuple(host(x) for x in l.quantized_cache.raw_bytes()) for l in m.full_layers()]
    for a, b in zip(before, after):
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)
    # restore assigns the length: a cleared cache comes back to the checkpoint's length,
    # over the rows still in the buffer
    for l in m.full_layers():
        l.clear_kv_cache()
    m.restore_cache(cps)
    assert [l.cache_seq_len() for l in m.full_layers()] == [12, 12]
    with pytest.raises(pk.KvCacheOverflow):
        m.full_layers()[0].quantized_cache.set_len(65)


def test_checkpoint_linear_state_roundtrip(pk):
    """A DeltaNet state checkpointed, stepped in place twice and restored equals the state
    at the checkpoint bit for bit; the step after the restore gives the same output as the
    first step after the checkpoint did."""
    say("rewind: DeltaNet state checkpoint / restore")
    m, g = make_model(pk, pk.KvCacheQuantization.Q4K)
    lin = [l for l in m.layers if isinstance(l, pk.LinearAttentionState)]
    at_cp = states(pk, m)
    cps = m.checkpoint_cache()
    g2 = torch.Generator(device="cuda").manual_seed(99)
    first = [host(step(l, g2)) for l in lin]
    for l in lin:
        step(l, g2)
    assert not np.array_equal(states(pk, m)[0][0], at_cp[0][0])
    m.restore_cache(cps)
    for a, b in zip(at_cp, states(pk, m)):
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)
    g2 = torch.Generator(device="cuda").manual_seed(99)
    again = [host(step(l, g2)) for l in lin]
    for a, b in zip(first, again):
        np.testing.assert_array_equal(a, b)
    # the backups were taken: a second restore leaves ssm / conv and sets the gate offset
    # to the (taken) backup's None, as RecurrentState::restore does (qn:746-757)
    m.restore_cache(cps)
    rs = lin[0].recurrent_state
    assert rs.gate_cumsum_offset is None and rs.backup_ssm is None
    # a checkpoint again reuses the buffers the restore kept: no new allocation
    spare = rs._spare[0]
    lin[0].checkpoint_state()
    assert rs.backup_ssm is spare


def test_checkpoint_without_state_and_cleared_state(pk):
    say("rewind: checkpoint with no state; state cleared before restore")
    m = pk.ModelKvState(4, 4, 16, 2, 256, 64, pk.KvCacheQuantization.Q4K)
    cps = m.checkpoint_cache()  # nothing created yet: Full{0} and markers
    assert [(c.kind, c.seq_len) for c in cps] == [("LinearAttention", 0)] * 3 + [("FullAttention", 0)]
    m.restore_cache(cps)
    m2, g = make_model(pk, pk.KvCacheQuantization.Q4K)
    cps = m2.checkpoint_cache()
    for l in m2.layers:
        if isinstance(l, pk.LinearAttentionState):
            l.clear_state()
    m2.restore_cache(cps)  # restore_state only acts on an existing state (qn:4021-4030)
    assert all(l.recurrent_state is None for l in m2.layers if isinstance(l, pk.LinearAttentionState))


def test_restore_to_intermediate_state(pk):
    say("rewind: restore_to_intermediate_state")
    m, _ = make_model(pk, pk.KvCacheQuantization.Q4K)
    before = states(pk, m)
    m.restore_to_intermediate_state(2, 6)  # full layers -> 6 + 2 + 1
    assert [l.cache_seq_len() for l in m.full_layers()] == [9, 9]
    for a, b in zip(before, states(pk, m)):  # no intermediate states held: unchanged
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)
