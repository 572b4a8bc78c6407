"""Helpers shared by the tests: exact float32 arithmetic for pinning the
oracle, and writers of hand-made indexes."""
from __future__ import annotations

import os
from fractions import Fraction

import numpy as np


def round_f32(x: Fraction) -> np.float32:
    """Correctly rounded (nearest, ties to even) float32 of an exact rational."""
    f = np.float32(float(x))
    best = None
    for c in (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))):
        err = abs(Fraction(float(c)) - x)
        if best is None or err < best[0] or (err == best[0] and (int(c.view(np.uint32)) & 1) == 0):
            best = (err, c)
    return np.float32(best[1])


def fma_f32(a, b, c) -> np.float32:
    return round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def add_f32(a, b) -> np.float32:
    return round_f32(Fraction(float(a)) + Fraction(float(b)))


def write_custom_index(d, X, adj, medoid, R, pq=None, nav=None):
    """Writes an index with an explicit adjacency (list of lists).  pq: a
    PQTables or None for an exact per-dim PQ (M = dim, pivots k, centroid 0);
    nav: (ids, adjacency, start) or None.  Returns (index, pq_prefix, nav_dir)."""
    from gustann_amd import index as gi
    os.makedirs(d, exist_ok=True)
    X = np.ascontiguousarray(X)
    n, dim = X.shape
    nbr = np.zeros((n, R), np.uint32)
    deg = np.zeros(n, np.uint32)
    for i, a in enumerate(adj):
        nbr[i, :len(a)] = a
        deg[i] = len(a)
    gi.write_disk_index(os.path.join(d, "x_disk.index"), X, nbr, deg, medoid)
    if pq is None:
        pq = exact_pq(X)
    gi.write_pq(os.path.join(d, "pq"), pq)
    nav_dir = ""
    if nav is not None:
        ids, nadj, start = nav
        nn = max(len(a) for a in nadj)
        nb = np.zeros((len(ids), nn), np.uint32)
        nd = np.zeros(len(ids), np.uint32)
        for i, a in enumerate(nadj):
            nb[i, :len(a)] = a
            nd[i] = len(a)
        nav_dir = os.path.join(d, "nav")
        gi.write_nav(nav_dir, np.ascontiguousarray(X[np.asarray(ids)]), nb, nd, start, np.asarray(ids))
    return os.path.join(d, "x_disk.index"), os.path.join(d, "pq"), nav_dir


def exact_pq(X):
    """PQ with one dim per chunk, pivots k = 0..255 and zero centroid: the
    codes are the coordinates and every LUT entry is an exact integer square."""
    from gustann_amd.index import PQTables
    X = np.asarray(X)
    n, dim = X.shape
    piv = np.repeat(np.arange(256, dtype=np.float32)[:, None], dim, axis=1)
    return PQTables(piv, np.zeros(dim, np.float32), np.arange(dim + 1, dtype=np.int32),
                    np.ascontiguousarray(X.astype(np.uint8)))


# A 12-node line graph worked by hand for the beam search: node i sits at
# x = BEAM_X[i] on the first axis (the other 3 dims 0), the query at the
# origin, the PQ exact (exact_pq), so every ADC and exact distance is x^2;
# entry node 0, list L = 4, top-3.  Each round takes the first `width`
# unvisited entries (marking them visited), then expands them in list order,
# each expansion inserting its unlisted neighbours (cut back to 4 entries)
# and pushing its own distance into the top-3.  The traces:
#   width 1 (the reference search): expands 0, 1, 3, 5, 7, 8 -> 6 expansions,
#     top-3 ids 8, 7, 5 (1, 4, 16);
#   width 2: rounds {0}, {1, 9}, {3, 2}, {5, 4}, {7, 6}, {8} -> 10 expansions,
#     top-3 ids 8, 7, 6 (1, 4, 9);
#   width 4: rounds {0}, {1, 9, 10}, {3, 2}, {5, 4}, {7, 6}, {8} -> 11
#     expansions, top-3 8, 7, 6.
# In the last round the list is [8, 7*, 6*, 5*] (width 2 and 4): a selection
# that did not mark its nodes visited would take 7 again.
BEAM_X = [10, 8, 7, 6, 5, 4, 3, 2, 1, 9, 11, 12]
BEAM_ADJ = [[1, 9, 10], [2, 3, 0], [4, 11], [5, 1], [6], [7, 2], [8], [8, 3], [7], [0, 2], [11], [10]]
BEAM_EXPECT = {1: (6, [8, 7, 5], [1.0, 4.0, 16.0]),
               2: (10, [8, 7, 6], [1.0, 4.0, 9.0]),
               4: (11, [8, 7, 6], [1.0, 4.0, 9.0])}


def write_beam_known_answer_index(d):
    X = np.zeros((len(BEAM_X), 4), np.uint8)
    X[:, 0] = BEAM_X
    return write_custom_index(d, X, BEAM_ADJ, 0, 3)
