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


def paged_plan(nblks, qis):
    """launch_paged_decode_q4k's stream plan (more than 32 pages): per workgroup its
    first segment and first slot; slots numbered piece by piece in workgroup order."""
    n, voff, V = len(nblks), [], 0
    for i, nb in enumerate(nblks):
        if i > 0:
            V += GAP
        voff.append(V)
        V += max(nb, 1)
    nwg = min(max((V + 3) // 4, 1), MAX_WGS)
    vq, vr = V // nwg, V % nwg
    wt, slot, sfirst = [], 0, 0
    nseq = max(qis) + 1
    wg0, wg1 = [-1] * nseq, [-1] * nseq
    for w in range(nwg):
        V0 = w * vq + min(w, vr)
        V1 = V0 + vq + (1 if w < vr else 0)
        while sfirst < n and voff[sfirst] + max(nblks[sfirst], 1) <= V0:
            sfirst += 1
        wt.append((sfirst, slot))
        i = sfirst
        while i < n and voff[i] < V1:
            if wg0[qis[i]] < 0:
                wg0[qis[i]] = slot
            slot += 1
            wg1[qis[i]] = slot
            i += 1
    return voff, nwg, vq, vr, wt, slot, wg0, wg1


def paged_pieces(nblks, voff, vq, vr, wt, w):
    """The kernel's scan over the device table (next_piece, dseg branch)."""
    V0 = w * vq + min(w, vr)
    V1 = V0 + vq + (1 if w < vr else 0)
    ps, slot = wt[w][0] - 1, wt[w][1] - 1
    out = []
    while True:
        for s in range(ps + 1, len(nblks)):
            if voff[s] >= V1:
                return out
            nb = nblks[s]
            ve = voff[s] + (nb if nb > 0 else 1)
            if ve > V0:
                ps, slot = s, slot + 1
                out.append((s, max(V0, voff[s]) - voff[s], min(min(V1, ve) - voff[s], nb), slot))
                break
        else:
            return out


def test_paged_plan_random():
    rng = random.Random(2)
    for _ in range(1500):
        nseq = rng.randint(1, 32)
        pblk = rng.choice([1, 4, 32, 128, 512])
        nblks, qis = [], []
        for q in range(nseq):
            for p in range(rng.randint(1, 12)):
                nblks.append(pblk)
                qis.append(q)
            nblks[-1] = rng.randint(0, pblk)  # the last page of a sequence is partly full
        if len(nblks) <= 32:
            continue
        voff, nwg, vq, vr, wt, nslots, wg0, wg1 = paged_plan(nblks, qis)
        cover = [[0] * nb for nb in nblks]
        seen = []
        for w in range(nwg):
            for s, b0, b1, slot in paged_pieces(nblks, voff, vq, vr, wt, w):
                seen.append((slot, qis[s]))
                for b in range(b0, b1):
                    cover[s][b] += 1
        assert all(c == 1 for row in cover for c in row)
        slots = [x[0] for x in seen]
        assert sorted(slots) == list(range(nslots))
        for q in range(max(qis) + 1):
            assert {sl for sl, qq in seen if qq == q} == set(range(wg0[q], wg1[q]))
