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
