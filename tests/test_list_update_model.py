"""The device list update (gustann_amd/csrc/gann_list.hpp list_plan /
list_apply) restated in Python, against the reference's formulation
(src/impl/pure_mem.cuh:350-419: merge with an equal new item after the old
one, cap at 2L, drop every entry whose id equals its predecessor's, cap at
L, take the first unvisited entry) on random update sequences.

The device form ranks each candidate in the list, drops candidates whose id
sits at their lower bound (duplicates) and candidates ranked at L (the list
is full and all of it orders below them), skips the sort when none is left,
places the k-th survivor in key order at rank + k, keeps the first L
entries, and picks min(new position of the old first-unvisited entry,
position of the first inserted entry).  Keys are the kernel's 64-bit
encoding: bits(dist) << 32 | id << 1 | visited.
"""
import bisect
import random

import pytest

VISITED = 1


def key_of(d, i):
    return (d << 32) | (i << 1)


def ident(k):
    return (k >> 1) & 0x7FFFFFFF


def reference_update(lst, cands, L):
    """Merge, 2L cap, adjacent-id dedup, L cap (pure_mem.cuh:350-419)."""
    merged = sorted([(k & ~VISITED, 0, k) for k in lst] + [(c, 1, c) for c in cands])
    merged = [t[2] for t in merged][:2 * L]
    out = []
    for k in merged:
        if out and ident(out[-1]) == ident(k):
            continue  # keeps the earlier (pre-existing) copy
        out.append(k)
    return out[:L]


def device_update(lst, cands, L, fu):
    """list_plan + list_apply of gann_list.hpp; returns (new list, next
    position or -1, the count of inserted entries, whether the sort ran)."""
    sz = len(lst)
    fu_entry = lst[fu] if fu < sz else None
    surv = []
    for c in cands:
        r = bisect.bisect_left(lst, c)           # entries ordered below c
        dup = r < sz and ident(lst[r]) == ident(c)
        if not dup and r < L:
            surv.append((c, r))
    sorted_run = bool(surv)
    surv.sort()
    nsz = min(sz + len(surv), L)
    pos = [r + e for e, (c, r) in enumerate(surv)]
    new = [None] * nsz
    marked = {p: c for p, (c, _) in zip(pos, surv) if p < nsz}
    nb = 0
    for j in range(nsz):                         # output j: inserted or old j - nb
        if j in marked:
            new[j] = marked[j]
            nb += 1
        else:
            new[j] = lst[j - nb]
    p0 = pos[0] if surv else None
    fu_new = None
    if fu < sz:
        fu_new = fu + sum(1 for (c, r) in surv if r <= fu)
    cands_pos = [x for x in (fu_new, p0) if x is not None]
    cand = min(cands_pos) if cands_pos else None
    if cand is None or cand >= nsz:
        return new, -1, len(surv), sorted_run
    sel = fu_entry if cand == fu_new else surv[0][0]
    assert new[cand] == sel
    return new, cand, len(surv), sorted_run


def first_unvisited(lst):
    for j, k in enumerate(lst):
        if not k & VISITED:
            return j
    return len(lst)


@pytest.mark.parametrize("L", [1, 4, 17, 64, 100, 300])
def test_device_update_equals_reference_merge(L):
    rng = random.Random(1000 + L)
    skipped = ran = 0
    for seq in range(60 if L < 100 else 25):
        ids = rng.sample(range(1, 5000), 600)
        dist = {i: rng.randrange(0, 40) for i in ids}  # few distinct values: many ties
        ref, dev = [], []
        fu = 0
        for step in range(80):
            deg = rng.randrange(0, 65)
            nbrs = rng.sample(ids, deg)                  # distinct ids, as in a record
            cands = [key_of(dist[i], i) for i in nbrs]
            ref = reference_update(ref, cands, L)
            dev, cand, n, sorted_run = device_update(dev, cands, L, fu)
            assert dev == ref, (L, seq, step)
            # the reference's next node: the first unvisited entry below L
            nxt = first_unvisited(ref)
            assert (cand if cand >= 0 else len(ref)) == nxt, (L, seq, step)
            skipped += not sorted_run
            ran += sorted_run
            if cand < 0:
                break
            ref[nxt] |= VISITED
            dev[cand] |= VISITED
            fu = first_unvisited(dev)
    assert ran > 0
    if L >= 17:
        assert skipped > 0  # the no-survivor path was exercised


def test_rank_at_L_is_never_inserted():
    """A full list and candidates that order after all of it: nothing is
    inserted, the sort is skipped, and the reference keeps the list too."""
    L = 8
    lst = [key_of(d, 100 + d) for d in range(L)]
    cands = [key_of(50 + j, 500 + j) for j in range(10)]
    new, cand, n, sorted_run = device_update(lst, cands, L, 0)
    assert n == 0 and not sorted_run and new == lst and cand == 0
    assert reference_update(lst, cands, L) == lst


def test_duplicate_of_the_last_entry_is_dropped():
    """The candidate equal to the unvisited last entry (same id, same
    distance) is a duplicate, not an insertion; a visited copy orders one
    above the fresh key and is found at the lower bound too."""
    L = 4
    lst = [key_of(d, 10 + d) for d in range(L)]
    for last in (lst[-1], lst[-1] | VISITED):
        cur = lst[:-1] + [last]
        new, _, n, _ = device_update(cur, [key_of(L - 1, 10 + L - 1)], L, 0)
        assert n == 0 and new == cur
        assert reference_update(cur, [key_of(L - 1, 10 + L - 1)], L) == cur


def device_rank(A, sz, key):
    """list_rank's index arithmetic (gann_list.hpp): a uniform first level of
    8 probes splitting A[0..sz) into 9 segments, then uniform steps inside
    the segment -- one binary step when the largest power of two within the
    segment's span is an odd power, 4-ary levels of 3 probes (reads clamped
    to the segment's end, probes at or past it count as not below) down to
    q = 4, and the level q = 1, which reads four entries from its lower bound
    clamped to sz - 1 and returns the one at the result.  Returns (rank,
    entry at min(rank, sz - 1) or None, reads after the first level)."""
    lo, end, span = 0, sz, sz
    if sz > 8:
        s = (sz + 8) // 9
        cnt = sum(1 for m in range(8) if A[min(s * (m + 1) - 1, sz - 1)] < key)
        lo = min(s * cnt, sz)
        end = sz if cnt == 8 else min(s * (cnt + 1) - 1, sz - 1)
        span = s
    if span <= 0:
        return 0, None, 0
    last, top = max(end - 1, 0), sz - 1
    lq = span.bit_length() - 1
    reads = 0
    if lq & 1:
        p = lo + (1 << lq) - 1
        if p < end and A[min(p, last)] < key:
            lo += 1 << lq
        reads += 1
        lq -= 1
    while lq >= 2:
        q = 1 << lq
        c = 0
        for j in (1, 2, 3):
            p = lo + j * q - 1
            c += 1 if (p < end and A[min(p, last)] < key) else 0
            reads += 1
        lo += c * q
        lq -= 2
    vals = [A[min(lo + j, top)] for j in range(4)]
    reads += 4
    c = sum(1 for j in range(3) if lo + j < end and vals[j] < key)
    return lo + c, vals[c], reads


@pytest.mark.parametrize("seed", range(6))
def test_device_rank_is_lower_bound(seed):
    # every size class of the first level and of the uniform steps, keys
    # below, between, equal to and above the entries
    rng = random.Random(seed)
    sizes = list(range(0, 70)) + [rng.randrange(70, 3000) for _ in range(60)] + [2575, 2576, 2624, 4096]
    for sz in sizes:
        A = sorted(rng.sample(range(0, 1 << 40, 2), sz))
        probes = [0, (1 << 40) + 1] + [rng.randrange(0, 1 << 40) for _ in range(20)]
        probes += [a for a in rng.sample(A, min(sz, 10))] + [a + 1 for a in rng.sample(A, min(sz, 10))]
        for key in probes:
            r, at_r, reads = device_rank(A, sz, key)
            assert r == bisect.bisect_left(A, key), (sz, key)
            if sz > 0:
                assert at_r == A[min(r, sz - 1)], (sz, key)
            if sz > 8:
                assert reads <= 16


def test_shift_windows_cover_the_changed_chunks():
    """list_apply's windows (gann_list.hpp): full 16-chunk windows from the top
    chunk ct down while chunks at or above cb (the first insertion's chunk)
    remain and the window fits above chunk 0, then windows of 8, 4, 2 and 1
    chunks under the same two conditions.  Every chunk from cb to ct is
    gathered exactly once, top window first; the windows stay inside
    [c0, ct], c0 = max(0, cb - 15), the chunks whose marks are cleared (those
    below cb copy onto themselves); at most 4 windows follow the 16-chunk
    ones."""
    for ct in range(0, 80):
        for cb in range(0, ct + 1):
            c0 = max(0, cb - 15)
            b_hi, wins = ct + 1, []
            while b_hi > cb and b_hi >= 16:
                wins.append((b_hi - 16, b_hi))
                b_hi -= 16
            n16 = len(wins)
            for kb in (8, 4, 2, 1):
                if b_hi > cb and b_hi >= kb:
                    wins.append((b_hi - kb, b_hi))
                    b_hi -= kb
            assert b_hi <= cb, (ct, cb)
            assert len(wins) - n16 <= 4
            covered = []
            for lo, hi in wins:
                assert c0 <= lo < hi <= ct + 1, (ct, cb, lo, hi)
                covered += list(range(hi - 1, lo - 1, -1))
            assert covered == sorted(covered, reverse=True)      # top down, no overlap
            assert set(range(cb, ct + 1)) <= set(covered)
            assert len(covered) == len(set(covered))
