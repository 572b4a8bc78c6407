"""The exact k-NN slice merge (gustann_amd/csrc/gann_knn.hip knn_merge_kernel
and launch_knn_merge) restated in Python: per query, slot a and slot
a + stride (a a multiple of 2 * stride, stride = 1, 2, 4, ...) merge into
slot a, entry j of A going to j + #{B < A[j]} and entry j of B to
j + #{A <= B[j]}, kept below k.  Checked against a sort of all slots'
entries: every slot count (odd ones included), padding entries (+inf, -1)
that tie with each other, real entries that tie in distance, and lists
shorter than k."""
import bisect
import random

import pytest

PAD = (0x7F800000 << 32) | 0xFFFFFFFF  # key of (+inf, -1)


def merge_pair(A, B, k):
    out = [None] * k
    for j, x in enumerate(A):
        r = j + bisect.bisect_left(B, x)
        if r < k:
            out[r] = x
    for j, y in enumerate(B):
        r = j + bisect.bisect_right(A, y)
        if r < k:
            out[r] = y
    return out


def merge_tree(slots, k):
    slots = [list(s) for s in slots]
    stride = 1
    while stride < len(slots):
        for a in range(0, len(slots), 2 * stride):
            b = a + stride
            if b < len(slots):
                slots[a] = merge_pair(slots[a], slots[b], k)
        stride *= 2
    return slots[0]


@pytest.mark.parametrize("k", [1, 3, 10, 100, 128])
def test_tree_merge_is_the_k_smallest(k):
    rng = random.Random(k)
    for trial in range(40):
        nslots = rng.randrange(1, 20)
        ids = rng.sample(range(1 << 20), nslots * k)
        slots, every = [], []
        for s in range(nslots):
            n = rng.randrange(0, k + 1)            # short lists pad with (+inf, -1)
            d = [rng.randrange(0, 30) for _ in range(n)]  # many equal distances
            keys = sorted((dd << 32) | ids[s * k + j] for j, dd in enumerate(d))
            every += keys
            slots.append(keys + [PAD] * (k - n))
        got = merge_tree(slots, k)
        want = sorted(every)[:k]
        assert got == want + [PAD] * (k - len(want)), (k, trial, nslots)


def compact_merge(buf, h, k):
    """knn_u8/f32 kernels' KnnBuf::compact, merge path (gann_knn.hip): the
    sorted prefix buf[:h] and at most 64 new keys buf[h:]; new key x goes to
    #{new < x} + #{old < x}, old key i to i + #{new < old i}; kept below k."""
    old, new = buf[:h], buf[h:]
    out = [None] * min(len(buf), k)
    for x in new:
        p = sum(1 for w in new if w < x) + bisect.bisect_left(old, x)
        if p < k:
            out[p] = x
    for i, o in enumerate(old):
        p = i + sum(1 for w in new if w < o)
        if p < k:
            out[p] = o
    return out


@pytest.mark.parametrize("k", [1, 2, 10, 64, 100, 128])
def test_compaction_merge_keeps_the_k_smallest(k):
    rng = random.Random(100 + k)
    for trial in range(300):
        h = rng.randrange(1, k + 1)                 # the kept, sorted prefix
        nn = rng.randrange(0, 65)                   # new keys since the last cut
        keys = rng.sample(range(1 << 40), h + nn)   # distinct, as (dist, id) keys are
        buf = sorted(keys[:h]) + keys[h:]
        assert compact_merge(buf, h, k) == sorted(keys)[:k], (k, trial)
