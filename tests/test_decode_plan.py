"""The stream-K partition of a batched decode launch, replayed in Python on random
segment sets: the formulas of launch_decode_segments (pkv_q4k_decode.hpp: virtual block
line with a gap before every segment after the first, workgroup ranges of vq or vq + 1
blocks, each segment's partial slots from the workgroups holding its first and last
virtual block) and of the kernel's piece scan (next_piece). Checked: every block of
every segment is processed by exactly one piece, piece slots are distinct and inside the
allocated nwg + n - 1, each segment's slot range [wg0, wg1) is exactly the set of its
pieces' slots (the combine reads nothing unwritten), and the segment's first workgroup
is the one that writes the prepared q. The GPU tests run the C++ plan and kernel against
the oracle (test_gpu_decode.py, test_gpu_prep.py)."""
import random

GAP = 6          # kPieceGap
MAX_WGS = 256    # kMainWGs


def plan(nblks):
    n, voff, V = len(nblks), [], 0
    for i, nb in enumerate(nblks):
        if i > 0:
            V += GAP
        voff.append(V)
        V += max(nb, 1)
    nwg = min(max((V + 3) // 4, 1), MAX_WGS)
    vq, vr = V // nwg, V % nwg

    def wg_of(x):
        big = vr * (vq + 1)
        return x // (vq + 1) if x < big else vr + (x - big) // vq

    first, wg0, wg1 = [], [], []
    for i in range(n):
        w0, w1 = wg_of(voff[i]), wg_of(voff[i] + max(nblks[i], 1) - 1)
        first.append(w0)
        wg0.append(w0 + i)
        wg1.append(w1 + i + 1)
    return voff, nwg, vq, vr, first, wg0, wg1


def pieces(nblks, voff, vq, vr, w):
    V0 = w * vq + min(w, vr)
    V1 = V0 + vq + (1 if w < vr else 0)
    out, ps = [], -1
    while True:
        for s in range(ps + 1, len(nblks)):
            vs = voff[s]
            if vs >= V1:
                return out
            nb = nblks[s]
            ve = vs + (nb if nb > 0 else 1)
            if ve > V0:
                ps = s
                out.append((s, max(V0, vs) - vs, min(min(V1, ve) - vs, nb), w + s))
                break
        else:
            return out


def check(nblks):
    n = len(nblks)
    voff, nwg, vq, vr, first, wg0, wg1 = plan(nblks)
    assert 1 <= nwg <= MAX_WGS and vq >= 1
    cover = [[0] * nb for nb in nblks]
    slots_of = [set() for _ in range(n)]
    all_slots = set()
    for w in range(nwg):
        for s, b0, b1, slot in pieces(nblks, voff, vq, vr, w):
            assert 0 <= slot < nwg + n - 1
            assert slot not in all_slots
            all_slots.add(slot)
            if not slots_of[s]:
                assert first[s] == w
            slots_of[s].add(slot)
            for b in range(b0, b1):
                cover[s][b] += 1
    for s in range(n):
        assert all(c == 1 for c in cover[s])
        assert slots_of[s] == set(range(wg0[s], wg1[s]))


def test_plan_examples():
    check([4096])            # config 3: 256 workgroups of 16 blocks
    check([0])
    check([1, 0, 0, 5])
    check([(S + 31) // 32 for S in (52614, 58721, 47995, 32578, 30468, 35753, 59532, 12849,
                                   27622, 62456, 31910, 49365, 41635, 45587, 53235, 28078)])
    voff, nwg, vq, vr, *_ = plan([4096])
    assert (nwg, vq, vr) == (256, 16, 0)


def test_plan_random():
    rng = random.Random(1)
    for _ in range(3000):
        n = rng.randint(1, 32)
        kind = rng.random()
        if kind < 0.3:
            nb = [rng.randint(0, 3) for _ in range(n)]
        elif kind < 0.6:
            nb = [rng.randint(0, 2100) for _ in range(n)]
        else:
            nb = [rng.choice([0, 1, 10, 33, 2048, 4096]) for _ in range(n)]
        check(nb)


def paged_plan(lens, fused, pblk):
    """launch_paged_decode_q4k's plan over device page lists: per sequence its virtual
    start, segment count (pages with keys; one virtual block for a fused step's sequence
    without keys), first segment index, and the combine's slot range."""
    pstride = pblk + GAP
    ptok = 32 * pblk
    pq, V, K = [], 0, 0
    for i, n in enumerate(lens):
        npg = -(-n // ptok) if n > 0 else 1
        if i > 0:
            V += GAP
        last = n - (npg - 1) * ptok
        nb_last = -(-last // 32)
        pq.append((n, V, npg, K))
        V += (npg - 1) * pstride + max(nb_last, 1)
        K += npg
    vend = []
    for i in range(len(lens)):
        n, vs, npg, kf = pq[i]
        last = n - (npg - 1) * ptok
        vend.append(vs + (npg - 1) * pstride + max(-(-last // 32), 1))
    nwg = min(max((V + 3) // 4, 1), MAX_WGS)
    vq, vr = V // nwg, V % nwg

    def wg_of(x):
        big = vr * (vq + 1)
        return x // (vq + 1) if x < big else vr + (x - big) // vq

    wg0 = [wg_of(pq[i][1]) + pq[i][3] for i in range(len(lens))]
    wg1 = [wg_of(vend[i] - 1) + pq[i][3] + pq[i][2] for i in range(len(lens))]
    return pq, nwg, vq, vr, K, pstride, ptok, wg0, wg1


def seg_keys(n, j, ptok):
    return min(n - j * ptok, ptok)


def paged_pieces(pq, nwg, vq, vr, pstride, ptok, w):
    """The kernel's scan (next_piece, kSegs == 0) and its empty-partial marker."""
    V0 = w * vq + min(w, vr)
    V1 = V0 + vq + (1 if w < vr else 0)
    nseq = len(pq)
    pi = 0
    while pi + 1 < nseq and pq[pi + 1][1] <= V0:
        pi += 1
    rel = V0 - pq[pi][1]
    pj = rel // pstride if rel > 0 else 0
    pj = min(pj, pq[pi][2] - 1)
    out = []
    while pi < nseq:
        n, vst, npg, kf = pq[pi]
        keys = seg_keys(n, pj, ptok)
        nb = -(-keys // 32)
        vs = vst + pj * pstride
        if vs >= V1:
            break
        ve = vs + max(nb, 1)
        k, i, j = kf + pj, pi, pj
        pj += 1
        if pj >= npg:
            pi, pj = pi + 1, 0
        if ve > V0:
            out.append((i, j, max(V0, vs) - vs, min(min(V1, ve) - vs, nb), w + k))
    # marker: the last segment starting before V1
    mi = 0
    while mi + 1 < nseq and pq[mi + 1][1] < V1:
        mi += 1
    n, vst, npg, kf = pq[mi]
    mj = min((V1 - 1 - vst) // pstride, npg - 1)
    nb = -(-seg_keys(n, mj, ptok) // 32)
    marker = w + kf + mj + 1 if vst + mj * pstride + max(nb, 1) <= V1 else None
    return out, marker


def test_paged_plan_random():
    rng = random.Random(2)
    for trial in range(1500):
        nseq = rng.randint(1, 32)
        pblk = rng.choice([1, 4, 32, 128, 512])
        fused = rng.random() < 0.5
        ptok = 32 * pblk
        lens = []
        for _ in range(nseq):
            r = rng.random()
            if r < 0.15 and fused:
                lens.append(0)
            elif r < 0.3:
                lens.append(rng.choice([1, ptok - 1, ptok, ptok + 1, 3 * ptok]))
            else:
                lens.append(rng.randint(1, 12 * ptok))
        pq, nwg, vq, vr, K, pstride, ptok, wg0, wg1 = paged_plan(lens, fused, pblk)
        cover = [[0] * -(-n // 32) for n in lens]
        written = {}
        for w in range(nwg):
            pieces, marker = paged_pieces(pq, nwg, vq, vr, pstride, ptok, w)
            for i, j, b0, b1, slot in pieces:
                assert slot not in written
                written[slot] = i
                for b in range(b0, b1):
                    cover[i][j * pblk + b] += 1
            if marker is not None:
                assert marker not in written
                written[marker] = None
        assert all(c == 1 for row in cover for c in row), trial
        assert all(0 <= sl < nwg + K for sl in written)
        for i in range(nseq):  # the combine's range: this row's pieces and empty partials only
            rng_slots = range(wg0[i], wg1[i])
            assert all(sl in written and written[sl] in (i, None) for sl in rng_slots), (trial, i)
            assert {sl for sl, q in written.items() if q == i} <= set(rng_slots)
