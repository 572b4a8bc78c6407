"""Writes the committed golden fixtures: two small indexes in the reference's
file formats and the oracle's outputs on them.

    python tests/golden/make_golden.py

Each fixture directory holds the index files exactly as the reference reads
them (disk index, PQ pivots and codes, pivot graph, query and ground-truth
vecs files; formats of src/layout.cpp:11-69, src/pq_search.cu:56-121,
src/nav_graph.cu:41-100, bin/utils.hpp:23-101) and `expected.npz`, computed
here by the CPU oracle (oracle/gann_oracle.c):

* `lut`        [nlut][M][256] f32  PQSearchData::init_query (src/impl/pq.cuh:8-59)
* `adc_ids`, `adc` [nq][S]         ADC sums (src/impl/pure_mem.cuh:300-310)
* `nav_local`, `entry` [nq]        get_entry_kernel + NavGraph::translate
                                   (src/impl/nav.cuh:13-135, src/nav_graph.cu:104-109)
* `s{L}_{k}_{nns,dists,found,nexp}` the fused search (src/impl/pure_mem.cuh:243-432)
                                   for each (L, k) in `search_cases`
* `b{W}_{L}_{k}_...`               the beam-width-W search mode of this library

The graph builder is multithreaded, so a rerun writes different (equally
valid) files; the fixtures are whatever was committed, and the tests check
every consumer against them.
"""
from __future__ import annotations

import json
import os
import shutil
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

# name -> (dataset spec keywords, number of LUTs kept, ADC ids per query,
#          (L, topk) search cases, (beam width, L, topk) beam cases)
FIXTURES = {
    "u8_small": (dict(n=1500, dim=32, dtype="uint8", nclusters=12, R=16, L_build=32, M=8, nq=48, k=10,
                      nav_n=150, nav_R=12, nav_L=24, pq_sample=1500, pq_iters=6, seed=4242),
                 2, 64, [(10, 10), (24, 5), (64, 10), (96, 32)], [(2, 24, 10), (4, 48, 10)]),
    "f32_small": (dict(n=800, dim=32, dtype="float", nclusters=10, sigma=0.3, R=16, L_build=32, M=16,
                       nq=40, k=10, nav_n=80, nav_R=12, nav_L=24, pq_sample=800, pq_iters=6, seed=777),
                  2, 64, [(10, 10), (32, 10), (64, 1)], [(3, 32, 10)]),
}


def make(name, out_root=HERE, threads=8):
    import oracle as orc
    from gustann_amd import index as gi
    kw, nlut, S, cases, beams = FIXTURES[name]
    d = os.path.join(out_root, name)
    if os.path.isdir(d):
        shutil.rmtree(d)
    meta = gi.build_dataset(gi.DatasetSpec(name=name, **kw), d, threads=threads)
    os.remove(os.path.join(d, "meta.json"))  # holds absolute paths; golden.json replaces it
    dtype = kw["dtype"]
    ix = orc.Index(os.path.join(d, "base_disk.index"), os.path.join(d, "pq"), os.path.join(d, "nav"),
                   dtype)
    qfile = os.path.join(d, "query." + ("bvecs" if dtype == "uint8" else "fvecs"))
    Q = gi.read_vecs(qfile, np.uint8 if dtype == "uint8" else np.float32).astype(np.float32)
    nq = Q.shape[0]
    out = {}
    out["lut"] = np.stack([orc.lut_build(ix.pivots, ix.centroid, ix.chunk_offsets, Q[i])
                           for i in range(nlut)])
    rng = np.random.default_rng(kw["seed"] + 99)
    ids = rng.integers(0, ix.num_pts, (nq, S)).astype(np.int32)
    out["adc_ids"] = ids
    out["adc"] = orc.adc_scan(ix.pivots, ix.centroid, ix.chunk_offsets, ix.codes, Q, ids, threads)
    nav = [ix.nav_entry_local(q)[0] for q in Q]
    ent = [ix.entry(q)[0] for q in Q]
    out["nav_local"] = np.asarray(nav, np.int32)
    out["entry"] = np.asarray(ent, np.int32)
    for L, k in cases:
        nns, dist, found, nexp, bad = ix.search(Q, k, L, threads=threads, check=True)
        if bad:
            raise RuntimeError(f"{name}: oracle invariant violations at L={L} k={k}")
        for key, v in (("nns", nns), ("dists", dist), ("found", found), ("nexp", nexp)):
            out[f"s{L}_{k}_{key}"] = v
    for w, L, k in beams:
        nns, dist, found, nexp = ix.search_beam(Q, k, L, w, threads=threads)
        for key, v in (("nns", nns), ("dists", dist), ("found", found), ("nexp", nexp)):
            out[f"b{w}_{L}_{k}_{key}"] = v
    np.savez_compressed(os.path.join(d, "expected.npz"), **out)
    spec = {"dtype": dtype, "dim": kw["dim"], "num_pts": int(ix.num_pts), "num_chunks": kw["M"],
            "medoid": int(ix.medoid), "nq": nq, "nlut": nlut, "adc_ids_per_query": S,
            "search_cases": [list(c) for c in cases], "beam_cases": [list(c) for c in beams],
            "files": {"index": "base_disk.index", "pq": "pq", "nav": "nav",
                      "query": os.path.basename(qfile), "gt": "gt.ivecs"},
            "generator": "tests/golden/make_golden.py (oracle/gann_oracle.c on index files written by "
                         "gustann_amd/csrc/index_builder.cpp)"}
    with open(os.path.join(d, "golden.json"), "w") as f:
        json.dump(spec, f, indent=1)
    return d


if __name__ == "__main__":
    for nm in (sys.argv[1:] or list(FIXTURES)):
        print(make(nm))
