"""Pins the oracle's beam search and pivot-graph entry search.

* The candidate-list semantics of src/impl/pure_mem.cuh:287-427 (merge with
  old-before-new ties, 2L cap, adjacent-duplicate removal, first unvisited
  below L, top-k insertion after equal values) are restated here with
  Python's sort instead of the reference's merge-path ranks, and the two
  formulations must agree exactly on random graphs.
* Known answers: a complete graph is visited entirely, with the entry node
  expanded twice; a complete pivot graph yields the exact nearest pivot; a
  hand-worked tie case and a degenerate two-node pivot graph follow the
  reference warp's shfl_down argmin and swap rules (src/impl/nav.cuh:84-133).
"""
import bisect
import os

import numpy as np
import pytest
from _helpers import exact_pq, write_custom_index

import oracle as orc
from gustann_amd import index as gi


def py_search(X, adj, pq, q, entry, topk, L):
    lut = orc.lut_build(pq.pivots, pq.centroid, pq.chunk_offsets, q)
    qr = orc.query_restore(pq.centroid, q)
    adc = lambda v: orc.adc(lut, pq.codes[v])
    lst = []  # [dist, id, visited]
    top = []
    u, nexp = entry, 0
    while u is not None:
        nexp += 1
        new = sorted((adc(v), int(v)) for v in adj[u])
        merged = sorted([(d, i, 0, vis) for d, i, vis in lst] + [(d, v, 1, False) for d, v in new],
                        key=lambda t: (t[0], t[1], t[2]))[:2 * L]
        ded = []
        for t in merged:
            if ded and ded[-1][1] == t[1]:
                continue
            ded.append(t)
        sel = next((k for k, t in enumerate(ded) if not t[3]), None)
        du = orc.l2(qr, X[u])
        top.insert(bisect.bisect_right([t[0] for t in top], du), (du, u))
        top = top[:topk]
        lst = [[t[0], t[1], t[3]] for t in ded[:L]]
        if sel is None or sel >= L:
            u = None
        else:
            lst[sel][2] = True
            u = lst[sel][1]
    return top, nexp


def random_graph(rng, n, R, min_deg=1):
    adj = []
    for u in range(n):
        k = int(rng.integers(min_deg, R + 1))
        cand = rng.choice(n - 1, size=k, replace=False)
        adj.append([int(c + (c >= u)) for c in cand])
    return adj


@pytest.mark.parametrize("seed,R,L,topk,trained,min_deg", [(0, 12, 4, 3, False, 1),
                                                           (1, 12, 8, 5, False, 1),
                                                           (2, 12, 16, 10, True, 1),
                                                           (3, 8, 24, 10, True, 1),
                                                           (4, 16, 6, 6, False, 1),
                                                           (5, 10, 40, 20, True, 1),
                                                           (6, 10, 12, 5, False, 0),
                                                           (7, 100, 40, 10, True, 1),
                                                           (8, 128, 150, 10, False, 60)])
def test_oracle_search_matches_sort_restatement(tmp_path, seed, R, L, topk, trained, min_deg):
    rng = np.random.default_rng(seed)
    n, D = 240, 16
    X = rng.integers(0, 256, (n, D)).astype(np.uint8)
    adj = random_graph(rng, n, R, min_deg=min_deg)
    pq = gi.train_pq(X, 4, sample=n, iters=4, seed=seed) if trained else exact_pq(X)
    idx, pqp, _ = write_custom_index(str(tmp_path), X, adj, 0, R, pq=pq)
    ix = orc.Index(idx, pqp)
    Q = rng.integers(0, 256, (12, D)).astype(np.float32)
    entries = rng.integers(0, n, 12).astype(np.int32)
    nns, dists, found, nexp, viol = ix.search(Q, topk, L, entries=entries, check=True)
    assert viol == 0
    for i in range(12):
        top, pe = py_search(X, adj, pq, Q[i], int(entries[i]), topk, L)
        assert found[i] == len(top)
        assert nexp[i] == pe
        assert [int(v) for v in nns[i, :found[i]]] == [t[1] for t in top]
        assert [float(v) for v in dists[i, :found[i]]] == [t[0] for t in top]
        assert np.all(nns[i, found[i]:] == 0) and np.all(dists[i, found[i]:] == 0)


def test_complete_graph_visits_everything_and_entry_twice(tmp_path):
    # Complete graph on n <= R nodes with L >= n: the entry is never in the
    # list, so it re-enters from its neighbours and is expanded (and
    # reranked) a second time; every other node is expanded once.
    n, D = 20, 8
    X = np.zeros((n, D), np.uint8)
    X[:, 0] = np.arange(n) * 3  # distinct exact distances to q
    q = np.zeros(D, np.float32)
    q[0] = 7.0
    adj = [[v for v in range(n) if v != u] for u in range(n)]
    idx, pqp, _ = write_custom_index(str(tmp_path), X, adj, 5, 24)
    ix = orc.Index(idx, pqp)
    nns, dists, found, nexp, viol = ix.search(q[None], 10, 32, check=True)
    assert viol == 0 and nexp[0] == n + 1
    d_all = sorted([(float((7 - 3 * i) ** 2), i) for i in range(n)] + [(float((7 - 15) ** 2), 5)])
    assert found[0] == 10
    assert [int(v) for v in nns[0]] == [i for _, i in d_all[:10]]
    assert [float(v) for v in dists[0]] == [d for d, _ in d_all[:10]]


def _nav_index(tmp_path, X, nadj, start, ids=None):
    n = X.shape[0]
    adj = [[(u + 1) % n] for u in range(n)]
    ids = list(range(n)) if ids is None else ids
    return write_custom_index(str(tmp_path), X, adj, 0, 4, nav=(ids, nadj, start))


def test_nav_complete_pivot_graph_finds_nearest(tmp_path):
    rng = np.random.default_rng(4)
    n, D = 25, 32
    X = rng.integers(0, 256, (n, D)).astype(np.uint8)
    nadj = [[v for v in range(n) if v != u] for u in range(n)]
    idx, pqp, nav = _nav_index(tmp_path, X, nadj, 3)
    ix = orc.Index(idx, pqp, nav)
    for _ in range(20):
        q = rng.integers(0, 256, D).astype(np.float32)
        d = ((X.astype(np.int64) - q.astype(np.int64)) ** 2).sum(1)
        if np.sum(d == d.min()) > 1:
            continue
        local, _ = ix.nav_entry_local(q)
        assert local == int(np.argmin(d))


def test_nav_tie_follows_shfl_down_tree(tmp_path):
    # Pivot 0 (start) links to 1, 2, 3 (slots 4, 5, 6); pivots 2 and 3 are at
    # the same distance 25 from q, pivot 1 at 36, pivot 0 at 100.  The argmin
    # tree of src/impl/nav.cuh:94-102 (strict '<', offsets 16..1) carries lane
    # 6 to lane 2 and lane 5 to lane 1 at offset 4; lane 0 takes lane 2 at
    # offset 2 and keeps it against lane 1 at offset 1: pivot 3 lands in slot
    # 0 and stays there.  A lowest-index or lowest-id argmin would give 2.
    D = 32
    X = np.full((4, D), 100, np.uint8)
    X[0, 2] = 110
    X[1, 0] = 106
    X[2, 0] = 105
    X[3, 1] = 105
    q = np.full(D, 100, np.float32)
    nadj = [[1, 2, 3], [0], [0], [0]]
    idx, pqp, nav = _nav_index(tmp_path, X, nadj, 0)
    ix = orc.Index(idx, pqp, nav)
    local, _ = ix.nav_entry_local(q)
    assert local == 3


def test_nav_two_node_graph_degenerates_to_empty_slot(tmp_path):
    # Two pivots linked to each other: after the second selection step only
    # +inf lanes remain, the tree keeps lane 0 and slot 2 swaps with slot 0
    # because their stored distances differ (src/impl/nav.cuh:105-116).  The
    # search ends with the empty id 0xffffffff in slot 0, i.e. pivot
    # 0x7fffffff, which the reference would look up out of bounds in
    # map.txt; the oracle (and the kernel) fall back to the medoid.
    D = 16
    X = np.full((2, D), 50, np.uint8)
    X[1, 0] = 52
    q = np.full(D, 50, np.float32)
    q[0] = 53.0  # pivot 1 is nearer than pivot 0
    idx, pqp, nav = _nav_index(tmp_path, X, [[1], [0]], 0)
    ix = orc.Index(idx, pqp, nav)
    local, _ = ix.nav_entry_local(q)
    assert local == 0x7FFFFFFF
    entry, fallback = ix.entry(q)
    assert fallback == 1 and entry == ix.medoid


def test_oracle_invariants_on_mixture(tiny_u8):
    P = tiny_u8["paths"]
    ix = orc.Index(P["index"], P["pq"], P["nav"])
    Q = gi.read_vecs(P["query"], np.uint8).astype(np.float32)[:60]
    gt = gi.read_vecs(P["gt"], np.int32)[:60]
    prev = -1.0
    for L in (10, 20, 40, 80):
        nns, dists, found, nexp, viol = ix.search(Q, 10, L, threads=4, check=True)
        assert viol == 0
        assert np.all(found == 10)
        # results are sorted by exact distance
        assert np.all(np.diff(dists, axis=1) >= 0)
        r = orc.recall(nns, gt, 10)
        assert r >= prev - 0.02  # recall grows with L (up to noise)
        prev = r
    assert prev > 0.8
