"""Index construction from a data file, in place of DiskANN's tools that the
reference's scripts call (absent here):

  * ``build_disk_index`` (scripts/build_diskann_index.sh:7):
    <prefix>_disk.index, <prefix>_pq_pivots.bin, <prefix>_pq_compressed.bin;
  * ``gen_small_file`` + ``build_memory_index`` + ``gen_tag.py``
    (scripts/gen_pivot_graph.sh:12-15): the pivot graph directory with
    nav_index, nav_index.data and map.txt;
  * optionally the exact ground truth of a query file (ivecs).

The flags follow build_disk_index's where they have a counterpart
(--data_type, --dist_fn, --index_path_prefix, --data_path, -R, -L, -B).
Vamana runs on the GPU for uint8 data (gann_build_vamana) or on the host;
the PQ codes are computed on the GPU (gann_pq_encode) or the host, with the
same result.  Data files: DiskANN .bin (int32 count, int32 dim, rows) or
bvecs / fvecs.

    python -m gustann_amd.build_disk_index --data_type uint8 --dist_fn l2 \\
        --index_path_prefix /data/idx --data_path /data/base.u8bin -R 64 -L 100 -B 3.2 \\
        --pivot_graph /data/nav --pivot_samples 1000000
    search_mem ... --index_path_prefix /data/idx --pq_path_prefix /data/idx_pq ...
"""
from __future__ import annotations

import argparse
import os
import sys
import time

import numpy as np

from . import index as gi


def read_data(path: str, data_type: str) -> np.ndarray:
    """Rows of a DiskANN .bin file (memory-mapped) or of a bvecs / fvecs file."""
    dt = np.uint8 if data_type == "uint8" else np.float32
    if path.endswith(("vecs",)):
        return gi.read_vecs(path, dt)
    head = np.fromfile(path, np.int32, count=2)
    if head.size != 2 or head[0] <= 0 or head[1] <= 0:
        raise ValueError(f"{path}: not a .bin file (int32 count, int32 dim, rows)")
    n, d = int(head[0]), int(head[1])
    if os.path.getsize(path) != 8 + n * d * np.dtype(dt).itemsize:
        raise ValueError(f"{path}: size does not match {n} rows of {d} {data_type}")
    return np.memmap(path, dtype=dt, mode="r", offset=8, shape=(n, d))


def pq_chunks_for_budget(n: int, dim: int, budget_gb: float) -> int:
    """Bytes of PQ code per point that fit the search memory budget (-B, GB),
    at most one chunk per dimension."""
    return int(max(1, min(dim, np.floor(budget_gb * (1 << 30) / max(n, 1)))))


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0],
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--data_type", choices=["uint8", "float"], required=True)
    ap.add_argument("--dist_fn", choices=["l2"], default="l2")
    ap.add_argument("--index_path_prefix", required=True)
    ap.add_argument("--data_path", required=True)
    ap.add_argument("-R", "--max_degree", type=int, default=64)
    ap.add_argument("-L", "--Lbuild", type=int, default=100)
    ap.add_argument("--alpha", type=float, default=1.2)
    ap.add_argument("-B", "--search_DRAM_budget", type=float, default=0.0,
                    help="GB for the PQ codes of all points (sets the chunk count)")
    ap.add_argument("--pq_chunks", type=int, default=0, help="PQ chunks (overrides -B)")
    ap.add_argument("-M", "--build_DRAM_budget", type=float, default=0.0, help="accepted, unused")
    ap.add_argument("--pq_sample", type=int, default=100_000)
    ap.add_argument("--builder", choices=["gpu", "cpu"], default="gpu",
                    help="graph and PQ encoding on the GPU (uint8 graphs only) or the host")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--pivot_graph", default="", help="directory for the pivot graph (nav index)")
    ap.add_argument("--pivot_samples", type=int, default=1_000_000)
    ap.add_argument("--query_path", default="")
    ap.add_argument("--gt_path", default="")
    ap.add_argument("--gt_k", type=int, default=100)
    a = ap.parse_args(argv)

    t0 = time.time()

    def log(msg):
        print(f"[build_disk_index {time.time() - t0:7.1f}s] {msg}", file=sys.stderr, flush=True)

    X = read_data(a.data_path, a.data_type)
    n, dim = X.shape
    M = a.pq_chunks or (pq_chunks_for_budget(n, dim, a.search_DRAM_budget) if a.search_DRAM_budget > 0
                        else min(dim, 32))
    gpu_graph = a.builder == "gpu" and a.data_type == "uint8"
    log(f"{n} x {dim} {a.data_type}; R={a.max_degree} L={a.Lbuild} alpha={a.alpha}; PQ {M} chunks; "
        f"graph on the {'GPU' if gpu_graph else 'host'}")
    if gpu_graph:
        nbr, deg, med = gi.build_vamana_gpu(X, a.max_degree, a.Lbuild, a.alpha, seed=a.seed, verbose=True)
    else:
        nbr, deg, med = gi.build_vamana(np.ascontiguousarray(X), a.max_degree, a.Lbuild, a.alpha, a.seed)
    log(f"graph: average degree {deg.mean():.1f}, medoid {med}")
    gi.write_disk_index(a.index_path_prefix + "_disk.index", X, nbr, deg, med)
    del nbr, deg
    pq = gi.train_pq(X, M, a.pq_sample, 12, a.seed + 1, encoder="gpu" if a.builder == "gpu" else "cpu")
    gi.write_pq(a.index_path_prefix + "_pq", pq)
    log(f"wrote {a.index_path_prefix}_disk.index and {a.index_path_prefix}_pq_{{pivots,compressed}}.bin")
    if a.pivot_graph:
        ns = min(a.pivot_samples, n)
        ids = gi.sample_ids(n, ns)
        Xs = np.ascontiguousarray(X[ids])
        if gpu_graph:
            nn, nd, nmed = gi.build_vamana_gpu(Xs, 32, 50, 1.2, seed=a.seed + 2)
        else:
            nn, nd, nmed = gi.build_vamana(Xs, 32, 50, 1.2, a.seed + 2)
        gi.write_nav(a.pivot_graph, Xs, nn, nd, nmed, ids)
        log(f"pivot graph of {ns} points in {a.pivot_graph}")
    if a.query_path and a.gt_path:
        Q = read_data(a.query_path, a.data_type).astype(np.float32)
        k = min(a.gt_k, n)
        if a.builder == "gpu":
            gt, _ = gi.brute_force_knn_gpu(X, Q, k)
        else:
            gt, _ = gi.brute_force_knn(np.ascontiguousarray(X), Q, k)
        gi.write_vecs(a.gt_path, gt)
        log(f"ground truth top-{k} of {Q.shape[0]} queries in {a.gt_path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
