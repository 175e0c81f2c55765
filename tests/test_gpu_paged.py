"""GPU parity of the paged KV caches (pkv_pool_* / pkv_seq_*): a pool of pages shared by
many sequences, against the CPU oracle's contiguous PreallocatedQuantizedKvCache
(qwen3_next.rs:343-643) on the same appended rows.

- Bytes: a sequence filled in chunks that cross page boundaries holds exactly the rows
  the oracle's cache holds (get_kv bit-exact), for every encoding.
- Decode (the model's shape, Q4K / Q8_0: one segment per page in the split-K decode
  kernels, kernel-argument and device segment tables) and prefill chunks / other shapes
  (rows gathered first) attend like the oracle (attn_checks' two gates); a batched varlen
  decode over several sequences matches each sequence alone.
- Sharing: a fork shares pages; appending into a shared, partly filled page copies it
  first, so neither sequence sees the other's rows; pages return to the pool.
- Rules: the cache offset rule (rewind / PKV_ERR_OFFSET), and pool exhaustion as
  PKV_ERR_OVERFLOW with nothing written."""
import sys

import numpy as np
import pytest

from attn_checks import assert_attn_close

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

F16, BF16, Q8_0, Q4K = 1, 2, 3, 4


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


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def fill(pk, orc, seq, cache, rng, chunks, H, D):
    for n in chunks:
        k = rng.standard_normal((1, H, n, D)).astype(np.float32)
        v = rng.standard_normal((1, H, n, D)).astype(np.float32)
        seq.append_quantized(dev(k), dev(v))
        assert cache.append(k, v) == 0


@pytest.mark.parametrize("quant,H,D,page", [(Q4K, 2, 256, 64), (Q8_0, 2, 256, 32),
                                            (F16, 4, 64, 128), (BF16, 1, 128, 32),
                                            (Q4K, 3, 200, 256)])
def test_bytes_match_oracle(pk, orc, quant, H, D, page):
    say(f"paged bytes quant={quant} H={H} D={D} page={page}")
    rng = np.random.default_rng(quant * 100 + page)
    pool = pk.PagedKvPool(H, D, page, 16, pk.KvCacheQuantization(quant))
    seq = pool.sequence()
    chunks = [37, page, 1, 90, 2 * page - 5]
    c = orc.Cache(quant, 1, H, D, sum(chunks))
    fill(pk, orc, seq, c, rng, chunks, H, D)
    assert seq.seq_len == sum(chunks) and seq.pages == -(-sum(chunks) // page)
    k, v = seq.get_kv()
    rk, rv = c.get_kv()
    assert np.array_equal(host(k), rk) and np.array_equal(host(v), rv)


def _attend(pk, orc, quant, H, Hkv, D, page, chunks, L, causal, seed, pool_pages=64):
    rng = np.random.default_rng(seed)
    pool = pk.PagedKvPool(Hkv, D, page, pool_pages, pk.KvCacheQuantization(quant))
    seq = pool.sequence()
    S = sum(chunks)
    c = orc.Cache(quant, 1, Hkv, D, S)
    fill(pk, orc, seq, c, rng, chunks, Hkv, D)
    q = rng.standard_normal((1, L, H, D)).astype(np.float32)
    scale = float(1 / np.sqrt(D))
    out = host(seq.attend(dev(q), scale, S - L, causal))
    ref = c.attend(q, scale, S - L, causal, mode="f64")
    assert_attn_close(out, ref, what=f"quant={quant} page={page} S={S} L={L}")
    return pool, seq


@pytest.mark.parametrize("quant,page,chunks", [
    (Q4K, 256, [1000]),              # 4 pages, last one partial: kernel-argument table
    (Q8_0, 256, [700, 300, 1]),
    (Q4K, 32, [2000, 21]),           # 64 pages: device segment table
    (Q8_0, 32, [1500]),              # 47 pages: device segment table
    (Q4K, 1024, [5000]),
    (Q4K, 64, [64]),                 # one full page
    (Q8_0, 128, [1]),                # one key
])
def test_decode_matches_oracle(pk, orc, quant, page, chunks):
    say(f"paged decode quant={quant} page={page} chunks={chunks}")
    _attend(pk, orc, quant, 16, 2, 256, page, chunks, 1, True, seed=sum(chunks) + page)


@pytest.mark.parametrize("quant,H,Hkv,D,page,chunks,L,causal", [
    (Q4K, 16, 2, 256, 256, [600, 64], 64, True),   # prefill chunk (gathered rows)
    (Q8_0, 16, 2, 256, 64, [300], 40, True),
    (F16, 4, 2, 64, 32, [257], 2, True),           # other shapes and encodings
    (Q8_0, 8, 8, 128, 64, [300], 3, False),
    (Q4K, 16, 2, 256, 128, [500], 1, False),        # decode without causality
])
def test_other_attends_match_oracle(pk, orc, quant, H, Hkv, D, page, chunks, L, causal):
    say(f"paged attend quant={quant} H={H}/{Hkv} D={D} page={page} L={L}")
    _attend(pk, orc, quant, H, Hkv, D, page, chunks, L, causal, seed=L + page)


@pytest.mark.parametrize("quant,page", [(Q4K, 256), (Q8_0, 128), (Q4K, 32)])
def test_batched_varlen_decode(pk, orc, quant, page):
    say(f"paged batched decode quant={quant} page={page}")
    rng = np.random.default_rng(7 + page)
    lens = [1, 31, 257, 1000, 70, 513, 32, 900]
    pool = pk.PagedKvPool(2, 256, page, sum(-(-n // page) for n in lens) + 2,
                          pk.KvCacheQuantization(quant))
    seqs, caches = [], []
    for n in lens:
        s = pool.sequence()
        c = orc.Cache(quant, 1, 2, 256, n)
        fill(pk, orc, s, c, rng, [n], 2, 256)
        seqs.append(s)
        caches.append(c)
    q = rng.standard_normal((len(lens), 16, 256)).astype(np.float32)
    out = host(pool.decode_batched(seqs, dev(q), 1 / 16))
    for i, (s, c) in enumerate(zip(seqs, caches)):
        ref = c.attend(q[i][None, None], 1 / 16, lens[i] - 1, True, mode="f64")[0, 0]
        assert_attn_close(out[i], ref, what=f"sequence {i} ({lens[i]} keys)")
        alone = host(s.attend(dev(q[i][None, None]), 1 / 16, lens[i] - 1))[0, 0]
        np.testing.assert_allclose(out[i], alone, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("quant", [Q4K, Q8_0])
def test_many_sequences_batched(pk, orc, quant):
    """40 sequences: two launches of at most 32 (Q4K: each over a device table, split
    stream-K over the pages)."""
    say(f"paged batched decode, 40 sequences, quant={quant}")
    rng = np.random.default_rng(40)
    lens = [int(x) for x in rng.integers(1, 300, 40)]
    pool = pk.PagedKvPool(2, 256, 64, sum(-(-n // 64) for n in lens), pk.KvCacheQuantization(quant))
    seqs, caches = [], []
    for n in lens:
        s = pool.sequence()
        c = orc.Cache(quant, 1, 2, 256, n)
        fill(pk, orc, s, c, rng, [n], 2, 256)
        seqs.append(s)
        caches.append(c)
    assert pool.free_pages == 0
    q = rng.standard_normal((40, 16, 256)).astype(np.float32)
    out = host(pool.decode_batched(seqs, dev(q), 1 / 16))
    for i in (0, 17, 31, 32, 39):
        ref = caches[i].attend(q[i][None, None], 1 / 16, lens[i] - 1, True, mode="f64")[0, 0]
        assert_attn_close(out[i], ref, what=f"sequence {i}")


@pytest.mark.parametrize("quant,page,nseq", [(Q4K, 32, 8), (Q4K, 256, 8), (Q8_0, 64, 8),
                                             (Q4K, 64, 40)])
def test_append_decode_batched(pk, orc, quant, page, nseq):
    """The fused step (pkv_seq_append_decode_batched) over empty, page-boundary and forked
    sequences, two steps in a row: each step's outputs against the oracle's attention over
    len + 1 keys, then every sequence's rows bit-exact to the oracle's cache. Q4K quantizes
    the new rows inside the decode launch; 40 sequences take two launches."""
    say(f"paged fused step quant={quant} page={page} sequences={nseq}")
    rng = np.random.default_rng(300 + page + nseq)
    base = [0, 1, page - 1, page, page + 1, 3 * page + 5, 700]
    lens = (base + [int(x) for x in rng.integers(1, 400, nseq)])[:nseq - 1]
    pool = pk.PagedKvPool(2, 256, page, sum(-(-(n + 2) // page) for n in lens) + 8 + 2 * nseq,
                          pk.KvCacheQuantization(quant))
    seqs, caches = [], []
    for n in lens:
        s = pool.sequence()
        c = orc.Cache(quant, 1, 2, 256, n + 2)
        if n:
            fill(pk, orc, s, c, rng, [n], 2, 256)
        seqs.append(s)
        caches.append(c)
    # a fork of the sequence whose last page is partly full: the step copies that page first
    src = 5 if nseq > 5 else 2
    f = seqs[src].fork()
    cf = orc.Cache(quant, 1, 2, 256, lens[src] + 2)
    cf.load_bytes(*caches[src].valid_bytes(), lens[src])
    seqs.append(f)
    caches.append(cf)
    for step in range(2):
        kn = rng.standard_normal((nseq, 2, 1, 256)).astype(np.float32)
        vn = rng.standard_normal((nseq, 2, 1, 256)).astype(np.float32)
        q = rng.standard_normal((nseq, 16, 256)).astype(np.float32)
        out = host(pool.append_decode_batched(seqs, dev(kn), dev(vn), dev(q), 1 / 16))
        for i, (s, c) in enumerate(zip(seqs, caches)):
            assert c.append(kn[i][None], vn[i][None]) == 0
            assert s.seq_len == c.seq_len
            ref = c.attend(q[i][None, None], 1 / 16, c.seq_len - 1, True, mode="f64")[0, 0]
            assert_attn_close(out[i], ref, what=f"step {step} sequence {i} ({c.seq_len} keys)")
    for i, (s, c) in enumerate(zip(seqs, caches)):
        k, v = s.get_kv()
        rk, rv = c.get_kv()
        assert np.array_equal(host(k), rk) and np.array_equal(host(v), rv), f"sequence {i}"
    assert pk.lib().pkv_device_status() == 0, pk.lib().pkv_last_error()


def test_fused_step_graph_replay(pk, orc):
    """A fused paged step whose sequences gain no page is captured in a HIP graph (Q4K
    page lists live on the device): three replays, with other eager work on the pool in
    between, each give the eager step's output bit for bit and leave the rows the oracle
    holds."""
    say("paged fused step, graph replay")
    rng = np.random.default_rng(12)
    lens = [100, 700, 33, 1500, 64 + 7]
    pool = pk.PagedKvPool(2, 256, 64, 64, pk.KvCacheQuantization.Q4K)
    seqs, caches = [], []
    for n in lens:
        s = pool.sequence()
        c = orc.Cache(Q4K, 1, 2, 256, n + 1)
        fill(pk, orc, s, c, rng, [n], 2, 256)
        seqs.append(s)
        caches.append(c)
    kn = dev(rng.standard_normal((5, 2, 1, 256)).astype(np.float32))
    vn = dev(rng.standard_normal((5, 2, 1, 256)).astype(np.float32))
    q = dev(rng.standard_normal((5, 16, 256)).astype(np.float32))
    outs = [None]

    def step():
        for s, n in zip(seqs, lens):
            s.truncate(n)
        outs[0] = pool.append_decode_batched(seqs, kn, vn, q, 1 / 16)

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()  # eager: sizes the workspace, syncs the page lists
        torch.cuda.synchronize()
        ref = host(outs[0])
        with torch.cuda.graph(graph, stream=side):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    got_out = outs[0]
    for i in range(3):
        other = pool.sequence()  # eager work on the pool between the replays
        other.append_quantized(kn[:1].repeat(1, 1, 3, 1), vn[:1].repeat(1, 1, 3, 1))
        torch.cuda.synchronize()
        del other
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(got_out), ref), f"replay {i}"
    for i, (s, c) in enumerate(zip(seqs, caches)):
        assert c.append(host(kn)[i][None], host(vn)[i][None]) == 0
        ref_i = c.attend(host(q)[i][None, None], 1 / 16, c.seq_len - 1, True, mode="f64")[0, 0]
        assert_attn_close(ref[i], ref_i, what=f"sequence {i}")
        k, v = s.get_kv()
        rk, rv = c.get_kv()
        assert np.array_equal(host(k), rk) and np.array_equal(host(v), rv), f"sequence {i}"


def test_append_decode_batched_all_or_nothing(pk, orc):
    """A pool one page short: PKV_ERR_OVERFLOW, no length or page changes."""
    say("paged fused step, pool overflow")
    rng = np.random.default_rng(8)
    pool = pk.PagedKvPool(2, 256, 32, 3, pk.KvCacheQuantization.Q4K)
    a, b = pool.sequence(), pool.sequence()
    ca, cb = orc.Cache(Q4K, 1, 2, 256, 64), orc.Cache(Q4K, 1, 2, 256, 64)
    fill(pk, orc, a, ca, rng, [32], 2, 256)   # one full page: the step needs a new one
    fill(pk, orc, b, cb, rng, [64], 2, 256)   # two full pages: so does this one
    assert pool.free_pages == 0
    kn = dev(rng.standard_normal((2, 2, 1, 256)).astype(np.float32))
    q = dev(rng.standard_normal((2, 16, 256)).astype(np.float32))
    with pytest.raises(pk.KvCacheOverflow):
        pool.append_decode_batched([a, b], kn, kn, q, 1 / 16)
    assert (a.seq_len, b.seq_len, a.pages, b.pages, pool.free_pages) == (32, 64, 1, 2, 0)


@pytest.mark.parametrize("quant", [Q4K, Q8_0])
def test_batched_decode_of_forks(pk, orc, quant):
    """Four sequences forked from one 1000-token prefix, each with its own suffix, decoded
    in one batched call: the shared pages appear once per sequence, so the launch lists
    more pages than the pool holds (the staging buffer grows)."""
    say(f"paged batched decode of forks, quant={quant}")
    rng = np.random.default_rng(77)
    pool = pk.PagedKvPool(2, 256, 32, 48, pk.KvCacheQuantization(quant))
    root = pool.sequence()
    croot = orc.Cache(quant, 1, 2, 256, 1000)
    fill(pk, orc, root, croot, rng, [1000], 2, 256)
    seqs, caches = [root], [croot]
    for i, extra in enumerate((5, 40, 90)):
        f = root.fork()
        c = orc.Cache(quant, 1, 2, 256, 1000 + extra)
        c.load_bytes(*croot.valid_bytes(), 1000)
        fill(pk, orc, f, c, rng, [extra], 2, 256)
        seqs.append(f)
        caches.append(c)
    assert sum(s.pages for s in seqs) > 48
    q = rng.standard_normal((4, 16, 256)).astype(np.float32)
    out = host(pool.decode_batched(seqs, dev(q), 1 / 16))
    for i, (s, c) in enumerate(zip(seqs, caches)):
        ref = c.attend(q[i][None, None], 1 / 16, s.seq_len - 1, True, mode="f64")[0, 0]
        assert_attn_close(out[i], ref, what=f"sequence {i} ({s.seq_len} keys)")


@pytest.mark.parametrize("quant", [Q4K, Q8_0])
def test_fork_copy_on_write(pk, orc, quant):
    say(f"paged fork / copy on write quant={quant}")
    rng = np.random.default_rng(99)
    pool = pk.PagedKvPool(2, 256, 64, 8, pk.KvCacheQuantization(quant))
    a = pool.sequence()
    ca = orc.Cache(quant, 1, 2, 256, 400)
    fill(pk, orc, a, ca, rng, [100], 2, 256)         # pages: one full, one with 36 rows
    assert pool.free_pages == 6
    b = a.fork()
    assert pool.free_pages == 6 and b.seq_len == 100 and b.pages == 2
    cb = orc.Cache(quant, 1, 2, 256, 400)
    cb.load_bytes(*ca.valid_bytes(), 100)
    fill(pk, orc, b, cb, rng, [10], 2, 256)           # copies the shared partial page
    assert pool.free_pages == 5
    fill(pk, orc, a, ca, rng, [50], 2, 256)           # a's page is its own again: no copy
    assert pool.free_pages == 4
    for s, c in ((a, ca), (b, cb)):
        k, v = s.get_kv()
        rk, rv = c.get_kv()
        assert np.array_equal(host(k), rk) and np.array_equal(host(v), rv)
    q = rng.standard_normal((1, 1, 16, 256)).astype(np.float32)
    for s, c in ((a, ca), (b, cb)):
        out = host(s.attend(dev(q), 1 / 16, s.seq_len - 1))
        assert_attn_close(out, c.attend(q, 1 / 16, s.seq_len - 1, True, mode="f64"))
    del s, b  # (the loop variable held b too)
    assert pool.free_pages == 5                       # b's own page back; page 0 still a's


def test_rules_offset_overflow_truncate_reuse(pk, orc):
    say("paged rules")
    rng = np.random.default_rng(5)
    pool = pk.PagedKvPool(2, 256, 32, 4, pk.KvCacheQuantization.Q4K)
    s = pool.sequence()
    c = orc.Cache(Q4K, 1, 2, 256, 128)
    fill(pk, orc, s, c, rng, [70], 2, 256)
    assert pool.free_pages == 1
    k = dev(rng.standard_normal((1, 2, 80, 256)).astype(np.float32))
    with pytest.raises(pk.KvCacheOverflow):
        s.append_quantized(k, k)                      # 150 tokens need 5 pages
    assert s.seq_len == 70 and pool.free_pages == 1  # nothing written
    with pytest.raises(pk.KvCacheOffsetMismatch):
        s.append_quantized(k[:, :, :1], k[:, :, :1], offset=71)
    # a smaller offset rewinds (the cache offset rule), then appends
    k2 = rng.standard_normal((1, 2, 5, 256)).astype(np.float32)
    s.append_quantized(dev(k2), dev(k2), offset=40)
    c.truncate(40)
    assert c.append(k2, k2) == 0
    assert s.seq_len == 45 and s.pages == 2 and pool.free_pages == 2
    got = host(s.get_kv()[0])
    assert np.array_equal(got, c.get_kv()[0])
    s.truncate(10)
    assert s.pages == 1 and pool.free_pages == 3
    del s                                             # every page back
    assert pool.free_pages == 4
    t = pool.sequence()                               # reused pages hold the new rows
    c2 = orc.Cache(Q4K, 1, 2, 256, 128)
    fill(pk, orc, t, c2, rng, [128], 2, 256)
    assert pool.free_pages == 0
    assert np.array_equal(host(t.get_kv()[1]), c2.get_kv()[1])


@pytest.mark.parametrize("quant", [Q4K, Q8_0, F16])
def test_append_batched_matches_single(pk, orc, quant):
    """One token into each of 5 sequences in one launch: a sequence at a page boundary, a
    forked pair sharing a partly filled page (each copies it first), an empty one."""
    say(f"paged batched append quant={quant}")
    rng = np.random.default_rng(123 + quant)
    pool = pk.PagedKvPool(2, 256, 32, 32, pk.KvCacheQuantization(quant))
    lens = [32, 40, 0, 5]
    seqs, caches = [], []
    for n in lens:
        s = pool.sequence()
        c = orc.Cache(quant, 1, 2, 256, 64)
        if n:
            fill(pk, orc, s, c, rng, [n], 2, 256)
        seqs.append(s)
        caches.append(c)
    fork = seqs[1].fork()  # shares seqs[1]'s page with 8 rows
    cf = orc.Cache(quant, 1, 2, 256, 64)
    cf.load_bytes(*caches[1].valid_bytes(), 40)
    seqs.append(fork)
    caches.append(cf)
    kn = rng.standard_normal((5, 2, 1, 256)).astype(np.float32)
    vn = rng.standard_normal((5, 2, 1, 256)).astype(np.float32)
    pool.append_batched(seqs, dev(kn), dev(vn))
    for i, (s, c) in enumerate(zip(seqs, caches)):
        assert c.append(kn[i:i + 1], vn[i:i + 1]) == 0
        assert s.seq_len == c.seq_len
        k, v = s.get_kv()
        rk, rv = c.get_kv()
        assert np.array_equal(host(k), rk) and np.array_equal(host(v), rv), i
    with pytest.raises(pk.KvCacheError):
        pool.append_batched([seqs[0], seqs[0]], dev(kn[:2]), dev(vn[:2]))


def test_refused_append_under_capture_changes_nothing(pk, orc):
    """An append whose page list would change (a copy on write of a shared, partly filled
    page, or a new page) is refused under graph capture before anything changes: page
    counts, free pages and lengths stay, and the next eager appends (a copy on write, then
    a smaller append) hold exactly the oracle's rows."""
    say("paged appends refused under capture")
    rng = np.random.default_rng(17)
    pool = pk.PagedKvPool(2, 256, 64, 8, pk.KvCacheQuantization.Q4K)
    a = pool.sequence()
    ca = orc.Cache(Q4K, 1, 2, 256, 400)
    fill(pk, orc, a, ca, rng, [100], 2, 256)  # one full page, one with 36 rows
    b = a.fork()
    cb = orc.Cache(Q4K, 1, 2, 256, 400)
    cb.load_bytes(*ca.valid_bytes(), 100)
    free0 = pool.free_pages
    k = rng.standard_normal((1, 2, 40, 256)).astype(np.float32)
    kn = rng.standard_normal((2, 2, 1, 256)).astype(np.float32)
    q = rng.standard_normal((2, 16, 256)).astype(np.float32)
    dk, dkn, dq = dev(k), dev(kn), dev(q)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    x = torch.zeros(1, device="cuda")
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            x.add_(1.0)
            with pytest.raises(pk.KvCacheError, match="graph"):
                b.append_quantized(dk, dk)  # copy on write + a new page
            with pytest.raises(pk.KvCacheError, match="graph"):
                pool.append_decode_batched([a, b], dkn, dkn, dq, 1 / 16)
    torch.cuda.synchronize()
    assert (a.seq_len, b.seq_len, a.pages, b.pages, pool.free_pages) == (100, 100, 2, 2, free0)
    b.append_quantized(dk, dk)  # eager: copies the shared page, takes a new one
    assert cb.append(k, k) == 0
    k2 = rng.standard_normal((1, 2, 3, 256)).astype(np.float32)
    b.append_quantized(dev(k2), dev(k2))
    assert cb.append(k2, k2) == 0
    assert pool.free_pages == free0 - 2
    for s, c in ((a, ca), (b, cb)):
        gk, gv = s.get_kv()
        rk, rv = c.get_kv()
        assert np.array_equal(host(gk), rk) and np.array_equal(host(gv), rv)


def test_graph_replay_survives_workspace_growth(pk, orc):
    """A captured fused paged step keeps working after an eager call on the same pool
    grows the pool's workspace (a 256-query prefill chunk needs far more split-K scratch
    than the decode): the buffer the graph's kernels write is retired, not freed, so the
    replays after the growth give the eager step's output bit for bit, and the chunk's
    own output matches the oracle."""
    say("paged graph replay after workspace growth")
    rng = np.random.default_rng(23)
    lens = [300, 1000]
    pool = pk.PagedKvPool(2, 256, 256, 16, pk.KvCacheQuantization.Q4K)
    seqs, caches = [], []
    for n in lens:
        s = pool.sequence()
        c = orc.Cache(Q4K, 1, 2, 256, n + 1)
        fill(pk, orc, s, c, rng, [n], 2, 256)
        seqs.append(s)
        caches.append(c)
    kn = dev(rng.standard_normal((2, 2, 1, 256)).astype(np.float32))
    q = dev(rng.standard_normal((2, 16, 256)).astype(np.float32))
    outs = [None]

    def step():
        for s, n in zip(seqs, lens):
            s.truncate(n)
        outs[0] = pool.append_decode_batched(seqs, kn, kn, q, 1 / 16)

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
        torch.cuda.synchronize()
        ref = host(outs[0])
        with torch.cuda.graph(graph, stream=side):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    got = outs[0]
    graph.replay()
    assert np.array_equal(host(got), ref)
    # eager prefill chunk over the longer sequence: grows the pool's workspace
    s1, n1 = seqs[1], lens[1]
    s1.truncate(n1)
    qc = rng.standard_normal((1, 256, 16, 256)).astype(np.float32)
    out_c = host(s1.attend(dev(qc), 1 / 16, n1 - 256))
    c1 = orc.Cache(Q4K, 1, 2, 256, n1)
    c1.load_bytes(*caches[1].valid_bytes(), n1)
    ref_c = c1.attend(qc, 1 / 16, n1 - 256, True, mode="f64")
    assert_attn_close(out_c, ref_c, what="prefill chunk after capture")
    for i in range(2):
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(got), ref), f"replay {i} after growth"
    assert pk.lib().pkv_device_status() == 0, pk.lib().pkv_last_error()
