"""Synthetic data, index building and file I/O in the reference's formats.

The reference builds its indexes with the external DiskANN tools
(scripts/build_diskann_index.sh:7, scripts/gen_pivot_graph.sh:12-14); this
module drives the package's own C++ builder (libgustann_index.so) and writes
the same files: <prefix>_disk.index, <pq>_pivots.bin, <pq>_compressed.bin,
nav/{nav_index, nav_index.data, map.txt}, plus bvecs/fvecs/ivecs for queries
and ground truth (bin/utils.hpp:23-88).
"""
from __future__ import annotations

import json
import os
from dataclasses import asdict, dataclass, field

import numpy as np

from ._native import icheck, index_lib

U8, F32 = 0, 1


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def _threads(n: int | None) -> int:
    return int(n or min(16, os.cpu_count() or 4))


# ------------------------------------------------------------------ data

def gen_mixture_u8(n, dim, nclusters, centre_seed, point_seed, lo=32.0, hi=224.0, sigma=12.0,
                   clusters=None, threads=None):
    """uint8 Gaussian mixture: centres ~ U[lo,hi]^dim, point = round(centre +
    N(0, sigma^2)) clipped to [0,255].  Returns (X [n,dim] u8, cluster ids)."""
    X = np.empty((n, dim), np.uint8)
    cid = np.empty(n, np.int32)
    cl = None if clusters is None else np.ascontiguousarray(clusters, np.int32)
    icheck(index_lib().gib_gen_mixture_u8(n, dim, nclusters, centre_seed, point_seed, lo, hi, sigma,
                                          _ptr(cl), _ptr(X), _ptr(cid), _threads(threads)))
    return X, cid


def gen_mixture_f32(n, dim, nclusters, centre_seed, point_seed, sigma, clusters=None, threads=None):
    """L2-normalised float mixture (centres ~ N(0,1) normalised)."""
    X = np.empty((n, dim), np.float32)
    cid = np.empty(n, np.int32)
    cl = None if clusters is None else np.ascontiguousarray(clusters, np.int32)
    icheck(index_lib().gib_gen_mixture_f32(n, dim, nclusters, centre_seed, point_seed, sigma,
                                           _ptr(cl), _ptr(X), _ptr(cid), _threads(threads)))
    return X, cid


def zipf_clusters(n, nclusters, s, seed):
    """Zipf(s) cluster ids (rejection-inversion, as bin/zipf.hpp)."""
    out = np.empty(n, np.int32)
    icheck(index_lib().gib_zipf_clusters(n, nclusters, s, seed, _ptr(out)))
    return out


# ------------------------------------------------------------------ builders

def build_vamana(X: np.ndarray, R: int, L: int, alpha=1.2, seed=1, threads=None):
    """Vamana graph over X.  Returns (nbr [n,R] u32, deg [n] u32, medoid)."""
    X = np.ascontiguousarray(X)
    n, dim = X.shape
    dtype = U8 if X.dtype == np.uint8 else F32
    nbr = np.zeros((n, R), np.uint32)
    deg = np.zeros(n, np.uint32)
    import ctypes
    med = ctypes.c_int64(0)
    icheck(index_lib().gib_vamana(_ptr(X), n, dim, dtype, R, L, alpha, seed, _threads(threads),
                                  _ptr(nbr), _ptr(deg), ctypes.byref(med)))
    return nbr, deg, int(med.value)


@dataclass
class PQTables:
    pivots: np.ndarray         # [256, dim] f32
    centroid: np.ndarray       # [dim] f32
    chunk_offsets: np.ndarray  # [M+1] i32
    codes: np.ndarray          # [n, M] u8

    @property
    def M(self):
        return int(self.chunk_offsets.shape[0] - 1)


def train_pq(X: np.ndarray, M: int, sample=100_000, iters=12, seed=2, threads=None,
             encoder: str = "cpu") -> PQTables:
    """k-means on a sample of X (host), then codes for every point on the
    host (encoder "cpu") or the GPU (encoder "gpu", gann_pq_encode: the
    same rule and arithmetic, so the same codes)."""
    X = np.ascontiguousarray(X)
    n, dim = X.shape
    dtype = U8 if X.dtype == np.uint8 else F32
    piv = np.empty((256, dim), np.float32)
    cen = np.empty(dim, np.float32)
    off = np.empty(M + 1, np.int32)
    codes = np.empty((n, M), np.uint8)
    if encoder == "gpu":
        icheck(index_lib().gib_pq_train(_ptr(X), n, dim, dtype, M, sample, iters, seed, _threads(threads),
                                        _ptr(piv), _ptr(cen), _ptr(off)))
        codes = pq_encode_gpu(X, piv, cen, off)
    else:
        icheck(index_lib().gib_pq(_ptr(X), n, dim, dtype, M, sample, iters, seed, _threads(threads),
                                  _ptr(piv), _ptr(cen), _ptr(off), _ptr(codes)))
    return PQTables(piv, cen, off, codes)


def pq_encode_gpu(X: np.ndarray, pivots, centroid, chunk_offsets, device_id: int = 0) -> np.ndarray:
    """PQ codes of X on the GPU (gann_pq_encode)."""
    from . import _native as N
    X = np.ascontiguousarray(X)
    if X.dtype != np.uint8:
        X = np.ascontiguousarray(X, np.float32)
    n, dim = X.shape
    piv = np.ascontiguousarray(pivots, np.float32)
    cen = np.ascontiguousarray(centroid, np.float32)
    off = np.ascontiguousarray(chunk_offsets, np.int32)
    M = off.shape[0] - 1
    codes = np.empty((n, M), np.uint8)
    N.check(N.hip_lib().gann_pq_encode(_ptr(X), n, dim, N.UINT8 if X.dtype == np.uint8 else N.FLOAT,
                                       _ptr(piv), _ptr(cen), _ptr(off), M, device_id, _ptr(codes)))
    return codes


def sample_ids(num_data: int, num_samp: int) -> np.ndarray:
    """bin/gen_small_file.cpp:18-25 sampling (mt19937(114514), shuffle, sort)."""
    out = np.empty(num_samp, np.int32)
    icheck(index_lib().gib_sample_ids(num_data, num_samp, _ptr(out)))
    return out


def brute_force_knn(X: np.ndarray, Q: np.ndarray, k: int, threads=None):
    """Exact squared-L2 k-NN (ties by smaller id).  Returns (ids, dists)."""
    X = np.ascontiguousarray(X)
    Q = np.ascontiguousarray(Q, np.float32)
    n, dim = X.shape
    dtype = U8 if X.dtype == np.uint8 else F32
    ids = np.empty((Q.shape[0], k), np.int32)
    d = np.empty((Q.shape[0], k), np.float32)
    icheck(index_lib().gib_brute_force(_ptr(X), n, _ptr(Q), Q.shape[0], dim, dtype, k, _ptr(ids),
                                       _ptr(d), _threads(threads)))
    return ids, d


def brute_force_knn_gpu(X: np.ndarray, Q: np.ndarray, k: int, device_id: int = 0):
    """The same exact k-NN on the GPU (gann_knn_exact: int8 MFMA for uint8 data,
    exact; fma chains for float).  Returns (ids, dists)."""
    from . import _native as N
    X = np.ascontiguousarray(X)
    Q = np.ascontiguousarray(Q, np.float32)
    n, dim = X.shape
    dtype = N.UINT8 if X.dtype == np.uint8 else N.FLOAT
    if dtype == N.FLOAT:
        X = np.ascontiguousarray(X, np.float32)
    ids = np.empty((Q.shape[0], k), np.int32)
    d = np.empty((Q.shape[0], k), np.float32)
    N.check(N.hip_lib().gann_knn_exact(_ptr(X), n, dim, dtype, _ptr(Q), Q.shape[0], k, device_id,
                                       _ptr(ids), _ptr(d)))
    return ids, d


def build_vamana_gpu(X: np.ndarray, R: int, L: int, alpha=1.2, seed=1, max_batch: int | None = None,
                     device_id: int = 0, verbose=False):
    """Vamana graph of uint8 points built on the GPU (gann_build_vamana):
    the host builder's steps with points inserted in batches of at most
    max_batch (default 0.5% of n, where recall over the built graph matched
    the host-built graph's at 10M points).  Returns (nbr [n,R] u32, deg [n] u32, medoid)."""
    import ctypes
    from . import _native as N
    X = np.ascontiguousarray(X)
    if X.dtype != np.uint8:
        raise ValueError("the GPU graph builder takes uint8 points")
    n, dim = X.shape
    if max_batch is None:
        max_batch = max(64, -(-n // 200))
    nbr = np.zeros((n, R), np.uint32)
    deg = np.zeros(n, np.uint32)
    med = ctypes.c_int64(0)
    N.check(N.hip_lib().gann_build_vamana(_ptr(X), n, dim, R, L, alpha, seed, max_batch, device_id,
                                          1 if verbose else 0, _ptr(nbr), _ptr(deg), ctypes.byref(med)))
    return nbr, deg, int(med.value)


def robust_prune_gpu(X: np.ndarray, p: int, cand, alpha: float, R: int, device_id: int = 0) -> np.ndarray:
    """One RobustPrune step of the GPU builder (gann_diag_robust_prune)."""
    import ctypes
    from . import _native as N
    X = np.ascontiguousarray(X, np.uint8)
    c = np.ascontiguousarray(cand, np.uint32)
    out = np.zeros(R, np.uint32)
    k = ctypes.c_int32(0)
    N.check(N.hip_lib().gann_diag_robust_prune(_ptr(X), X.shape[0], X.shape[1], p, _ptr(c), c.shape[0],
                                               alpha, R, device_id, _ptr(out), ctypes.byref(k)))
    return out[:k.value].copy()


# ------------------------------------------------------------------ writers

def write_disk_index(path, X, nbr, deg, medoid):
    X = np.ascontiguousarray(X)
    nbr = np.ascontiguousarray(nbr, np.uint32)
    deg = np.ascontiguousarray(deg, np.uint32)
    n, dim = X.shape
    icheck(index_lib().gib_write_disk_index(os.fsencode(path), _ptr(X), n, dim, X.itemsize,
                                            nbr.shape[1], medoid, _ptr(nbr), _ptr(deg)))


def write_pq(prefix, pq: PQTables):
    piv = np.ascontiguousarray(pq.pivots, np.float32)
    cen = np.ascontiguousarray(pq.centroid, np.float32)
    off = np.ascontiguousarray(pq.chunk_offsets, np.int32)
    codes = np.ascontiguousarray(pq.codes, np.uint8)
    icheck(index_lib().gib_write_pq(os.fsencode(prefix), _ptr(piv), _ptr(cen), _ptr(off),
                                    piv.shape[1], off.shape[0] - 1, _ptr(codes), codes.shape[0]))


def write_nav(dirpath, Xs, nbr, deg, start, mapping):
    os.makedirs(dirpath, exist_ok=True)
    Xs = np.ascontiguousarray(Xs)
    nbr = np.ascontiguousarray(nbr, np.uint32)
    deg = np.ascontiguousarray(deg, np.uint32)
    mapping = np.ascontiguousarray(mapping, np.int32)
    n, dim = Xs.shape
    icheck(index_lib().gib_write_nav(os.fsencode(dirpath), _ptr(Xs), n, dim, Xs.itemsize,
                                     _ptr(nbr), _ptr(deg), nbr.shape[1], start, _ptr(mapping)))


def write_vecs(path, A):
    A = np.ascontiguousarray(A)
    icheck(index_lib().gib_write_vecs(os.fsencode(path), A.itemsize, A.shape[0], A.shape[1],
                                      _ptr(A)))


def inspect(index_file, pq_prefix, nav_prefix="", elem_size=1):
    """Parses an index with the C++ readers of the search library; returns a
    dict of its layout or raises RuntimeError with the reader's message."""
    out = np.zeros(12, np.int64)
    icheck(index_lib().gib_inspect(os.fsencode(index_file), os.fsencode(pq_prefix),
                                   os.fsencode(nav_prefix) if nav_prefix else None, elem_size,
                                   _ptr(out)))
    keys = ("num_pts", "dim", "medoid", "node_len", "nodes_per_page", "max_m", "num_pages",
            "pq_dim", "pq_num_chunks", "pq_num_pts", "nav_num_node", "nav_max_m")
    return dict(zip(keys, (int(v) for v in out)))


def read_pq(prefix):
    """<pq>_pivots.bin + <pq>_compressed.bin (src/pq_search.cu:56-121) as a
    PQTables (legacy nr = 5 offset tables read chunk offsets from slot 3)."""
    def bin_at(path, off, dt):
        with open(path, "rb") as f:
            f.seek(off)
            n, d = np.frombuffer(f.read(8), np.int32)
            a = np.frombuffer(f.read(int(n) * int(d) * np.dtype(dt).itemsize), dt)
        return a.reshape(int(n), int(d))
    pv = prefix + "_pivots.bin"
    offs = bin_at(pv, 0, np.uint64).ravel()
    if offs.shape[0] not in (4, 5):
        raise ValueError("pq pivots: offset table must be 4x1 or 5x1")
    piv = bin_at(pv, int(offs[0]), np.float32)
    cen = bin_at(pv, int(offs[1]), np.float32).ravel()
    co = bin_at(pv, int(offs[3 if offs.shape[0] == 5 else 2]), np.int32).ravel()
    codes = bin_at(prefix + "_compressed.bin", 0, np.uint8)
    return PQTables(piv.copy(), cen.copy(), co.copy(), codes.copy())


def read_pq_meta(prefix):
    """(dim, num_chunks) of a PQ pivots file without reading the codes."""
    pv = prefix + "_pivots.bin"
    with open(pv, "rb") as f:
        n, _ = np.frombuffer(f.read(8), np.int32)
        offs = np.frombuffer(f.read(8 * int(n)), np.uint64)
        f.seek(int(offs[0]))
        _, dim = np.frombuffer(f.read(8), np.int32)
        f.seek(int(offs[3 if int(n) == 5 else 2]))
        m1, _ = np.frombuffer(f.read(8), np.int32)
    return int(dim), int(m1) - 1


def read_vecs(path, dtype):
    """bvecs (uint8) / fvecs (float32) / ivecs (int32) reader (bin/utils.hpp:23-88)."""
    raw = np.fromfile(path, np.uint8)
    if raw.size == 0:
        raise ValueError(f"empty vecs file {path}")
    d = int(np.frombuffer(raw[:4].tobytes(), np.int32)[0])
    item = np.dtype(dtype).itemsize
    row = 4 + d * item
    if d <= 0 or raw.size % row:
        raise ValueError(f"weird file size for {path}")
    rows = raw.reshape(-1, row)
    if not np.all(rows[:, :4].copy().view(np.int32).ravel() == d):
        raise ValueError(f"inconsistent row dimension in {path}")
    return np.ascontiguousarray(rows[:, 4:]).view(dtype).reshape(-1, d)


# ------------------------------------------------------------------ datasets

@dataclass
class DatasetSpec:
    """One synthetic workload: base set, queries, index and PQ parameters."""
    name: str
    n: int
    dim: int
    dtype: str = "uint8"          # "uint8" | "float"
    nclusters: int = 1000
    sigma: float = 12.0
    lo: float = 32.0
    hi: float = 224.0
    R: int = 64
    L_build: int = 100
    alpha: float = 1.2
    M: int = 32
    pq_sample: int = 100_000
    pq_iters: int = 12
    nq: int = 1000
    k: int = 10
    nav_n: int = 0                # 0 = no pivot graph
    nav_R: int = 32
    nav_L: int = 50
    zipf_s: float = 0.0           # > 0: query clusters ~ Zipf(s)
    gt_nq: int = 0                # ground truth for the first gt_nq queries (0 = all)
    seed: int = 1234
    builder: str = "cpu"          # "cpu": host Vamana + host ground truth; "gpu": both on the GPU (uint8)
    # more query sets over the same index: {"name", "nq", "zipf_s", "k", "gt_nq"}
    extra_queries: list = field(default_factory=list)
    extra: dict = field(default_factory=dict)


def build_dataset(spec: DatasetSpec, out_dir: str, threads=None, verbose=False) -> dict:
    """Generates data, builds the Vamana graph, PQ and (optionally) the pivot
    graph, computes ground truth and writes everything under out_dir.
    Returns a dict of paths and metadata (also saved as meta.json)."""
    import sys
    import time
    os.makedirs(out_dir, exist_ok=True)
    index_lib().gib_set_verbose(1 if verbose else 0)
    t0 = time.time()
    s = spec.seed
    if spec.dtype == "uint8":
        X, _ = gen_mixture_u8(spec.n, spec.dim, spec.nclusters, s, s + 1, spec.lo, spec.hi, spec.sigma,
                              threads=threads)
        qcl = zipf_clusters(spec.nq, spec.nclusters, spec.zipf_s, s + 7) if spec.zipf_s > 0 else None
        Qb, _ = gen_mixture_u8(spec.nq, spec.dim, spec.nclusters, s, s + 2, spec.lo, spec.hi,
                               spec.sigma, clusters=qcl, threads=threads)
        Q = Qb.astype(np.float32)
    else:
        X, _ = gen_mixture_f32(spec.n, spec.dim, spec.nclusters, s, s + 1, spec.sigma, threads=threads)
        qcl = zipf_clusters(spec.nq, spec.nclusters, spec.zipf_s, s + 7) if spec.zipf_s > 0 else None
        Q, _ = gen_mixture_f32(spec.nq, spec.dim, spec.nclusters, s, s + 2, spec.sigma, clusters=qcl,
                               threads=threads)
        Qb = Q
    if verbose:
        print(f"[{spec.name}] data {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    gpu = spec.builder == "gpu"
    if gpu and spec.dtype != "uint8":
        raise ValueError("the GPU graph builder takes uint8 data")
    if gpu:
        nbr, deg, med = build_vamana_gpu(X, spec.R, spec.L_build, spec.alpha, s + 3, verbose=verbose)
    else:
        nbr, deg, med = build_vamana(X, spec.R, spec.L_build, spec.alpha, s + 3, threads)
    if verbose:
        print(f"[{spec.name}] vamana {time.time() - t0:.1f}s (avg deg {deg.mean():.1f})", file=sys.stderr,
              flush=True)
    pq = train_pq(X, spec.M, spec.pq_sample, spec.pq_iters, s + 4, threads, encoder="gpu" if gpu else "cpu")
    if verbose:
        print(f"[{spec.name}] pq {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    ngt = spec.gt_nq if spec.gt_nq > 0 else spec.nq
    if gpu:
        gt, gtd = brute_force_knn_gpu(X, Q[:ngt], max(spec.k, 10))
    else:
        gt, gtd = brute_force_knn(X, Q[:ngt], max(spec.k, 10), threads)
    if verbose:
        print(f"[{spec.name}] gt {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    paths = {
        "index": os.path.join(out_dir, "base_disk.index"),
        "pq": os.path.join(out_dir, "pq"),
        "nav": os.path.join(out_dir, "nav") if spec.nav_n > 0 else "",
        "query": os.path.join(out_dir, "query." + ("bvecs" if spec.dtype == "uint8" else "fvecs")),
        "gt": os.path.join(out_dir, "gt.ivecs"),
    }
    write_disk_index(paths["index"], X, nbr, deg, med)
    avg_deg = float(deg.mean())
    del nbr, deg
    write_pq(paths["pq"], pq)
    write_vecs(paths["query"], Qb)
    write_vecs(paths["gt"], gt)
    for xi, xq in enumerate(spec.extra_queries):
        nm = xq["name"]
        zs = float(xq.get("zipf_s", 0.0))
        xcl = zipf_clusters(int(xq["nq"]), spec.nclusters, zs, s + 17 + xi) if zs > 0 else None
        if spec.dtype == "uint8":
            xQb, _ = gen_mixture_u8(int(xq["nq"]), spec.dim, spec.nclusters, s, s + 19 + xi, spec.lo, spec.hi,
                                    spec.sigma, clusters=xcl, threads=threads)
            xQ = xQb.astype(np.float32)
        else:
            xQ, _ = gen_mixture_f32(int(xq["nq"]), spec.dim, spec.nclusters, s, s + 19 + xi, spec.sigma,
                                    clusters=xcl, threads=threads)
            xQb = xQ
        xk = max(int(xq.get("k", 10)), 10)
        xg = int(xq.get("gt_nq", 0)) or xQ.shape[0]
        if gpu:
            xgt, _ = brute_force_knn_gpu(X, xQ[:xg], xk)
        else:
            xgt, _ = brute_force_knn(X, xQ[:xg], xk, threads)
        paths[f"query_{nm}"] = os.path.join(out_dir, f"query_{nm}." + ("bvecs" if spec.dtype == "uint8" else "fvecs"))
        paths[f"gt_{nm}"] = os.path.join(out_dir, f"gt_{nm}.ivecs")
        write_vecs(paths[f"query_{nm}"], xQb)
        write_vecs(paths[f"gt_{nm}"], xgt)
    if verbose:
        print(f"[{spec.name}] written {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    if spec.nav_n > 0:
        ids = sample_ids(spec.n, spec.nav_n)
        Xs = np.ascontiguousarray(X[ids])
        if gpu:
            nn, nd, nmed = build_vamana_gpu(Xs, spec.nav_R, spec.nav_L, 1.2, s + 5)
        else:
            nn, nd, nmed = build_vamana(Xs, spec.nav_R, spec.nav_L, 1.2, s + 5, threads)
        write_nav(paths["nav"], Xs, nn, nd, nmed, ids)
        if verbose:
            print(f"[{spec.name}] pivot graph {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    meta = {"spec": asdict(spec), "paths": paths, "medoid": med,
            "avg_degree": avg_deg, "build_s": time.time() - t0,
            "rng": "splitmix64-seeded xoshiro256** streams per point, Box-Muller normals"}
    with open(os.path.join(out_dir, "meta.json"), "w") as f:
        json.dump(meta, f, indent=1)
    return meta
