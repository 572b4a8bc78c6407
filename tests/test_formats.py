"""Reference file formats: writers and the C++ readers shared with the search
library (formats.hpp) round-trip, and malformed files are rejected with an
error instead of the reference's exit()/abort() (src/layout.cpp:11-69,
src/pq_search.cu:56-121, src/nav_graph.cu:41-100, bin/utils.hpp:23-88)."""
import os
import struct

import numpy as np
import pytest
from _helpers import write_custom_index

from gustann_amd import index as gi


def _records(index_file, dim, elem=1):
    meta = np.fromfile(index_file, np.uint64, count=8, offset=8)
    n, d, med, node_len, npp = (int(v) for v in meta[:5])
    pages = np.fromfile(index_file, np.uint8, offset=4096)
    out = []
    for u in range(n):
        off = (u // npp) * 4096 + (u % npp) * node_len
        rec = pages[off:off + node_len]
        coords = rec[:dim * elem]
        deg = int(rec[dim * elem:dim * elem + 4].view(np.uint32)[0])
        nbrs = rec[dim * elem + 4:dim * elem + 4 + 4 * deg].view(np.uint32)
        out.append((coords, list(nbrs)))
    return out


def test_disk_index_roundtrip(tmp_path):
    rng = np.random.default_rng(0)
    X = rng.integers(0, 256, (333, 20)).astype(np.uint8)
    adj = [list(rng.choice(332, size=int(rng.integers(0, 9)), replace=False)) for _ in range(333)]
    adj = [[int(v + (v >= u)) for v in a] for u, a in enumerate(adj)]
    idx, pqp, _ = write_custom_index(str(tmp_path), X, adj, 17, 8)
    info = gi.inspect(idx, pqp)
    assert info["num_pts"] == 333 and info["dim"] == 20 and info["medoid"] == 17
    assert info["max_m"] == 8 and info["node_len"] == 20 + 4 * 9
    assert info["nodes_per_page"] == 4096 // 56 and info["num_pages"] == -(-333 // (4096 // 56))
    for u, (c, nb) in enumerate(_records(idx, 20)):
        assert np.array_equal(c, X[u]) and nb == adj[u]


def test_float_index_and_pq_roundtrip(tmp_path):
    rng = np.random.default_rng(1)
    X = rng.normal(size=(500, 24)).astype(np.float32)
    pq = gi.train_pq(X, 6, sample=500, iters=3)
    idx = str(tmp_path / "f_disk.index")
    nbr, deg, med = gi.build_vamana(X, 8, 16, seed=3)
    gi.write_disk_index(idx, X, nbr, deg, med)
    gi.write_pq(str(tmp_path / "pq"), pq)
    info = gi.inspect(idx, str(tmp_path / "pq"), elem_size=4)
    assert info["dim"] == 24 and info["pq_num_chunks"] == 6 and info["pq_num_pts"] == 500
    back = gi.read_pq(str(tmp_path / "pq"))
    for a, b in ((back.pivots, pq.pivots), (back.centroid, pq.centroid),
                 (back.chunk_offsets, pq.chunk_offsets), (back.codes, pq.codes)):
        assert np.array_equal(a, b)
    for u, (c, nb) in enumerate(_records(idx, 24, 4)):
        assert np.array_equal(c.view(np.float32), X[u]) and nb == list(nbr[u, :deg[u]])


def _write_pivots_file(path, sections, nr):
    """Offset table of nr u64 entries at 0, sections back to back from 4096."""
    offs = []
    blob = b""
    pos = 4096
    for arr in sections:
        data = struct.pack("<ii", arr.shape[0], arr.shape[1]) + arr.tobytes()
        offs.append(pos)
        blob += data
        pos += len(data)
    offs.append(pos)
    offs = offs[:nr]
    with open(path, "wb") as f:
        f.write(struct.pack("<ii", nr, 1) + np.array(offs, np.uint64).tobytes())
        f.seek(4096)
        f.write(blob)


def test_legacy_pivots_layout_reads_chunk_offsets_from_slot_3(tmp_path):
    # nr == 5: [pivots, centroid, rearrangement, chunk_offsets, end]
    # (src/pq_search.cu:98-107); the rearrangement is ignored.
    rng = np.random.default_rng(2)
    D, M = 12, 4
    X = rng.integers(0, 256, (50, D)).astype(np.uint8)
    idx, pqp, _ = write_custom_index(str(tmp_path), X, [[(u + 1) % 50] for u in range(50)], 0, 2)
    piv = rng.normal(size=(256, D)).astype(np.float32)
    cen = rng.normal(size=(D, 1)).astype(np.float32)
    rearr = np.arange(D, dtype=np.int32)[::-1].reshape(D, 1).copy()
    off = np.arange(0, D + 1, 3, dtype=np.int32).reshape(M + 1, 1)
    _write_pivots_file(pqp + "_pivots.bin", [piv, cen, rearr, off], 5)
    with open(pqp + "_compressed.bin", "wb") as f:
        f.write(struct.pack("<ii", 50, M) + rng.integers(0, 256, (50, M)).astype(np.uint8).tobytes())
    info = gi.inspect(idx, pqp)
    assert info["pq_num_chunks"] == M
    back = gi.read_pq(pqp)
    assert np.array_equal(back.chunk_offsets, off.ravel()) and np.array_equal(back.pivots, piv)


@pytest.mark.parametrize("case", ["nr3", "pivots255", "chunks_short", "chunks_decreasing",
                                  "codes_mismatch", "index_truncated", "missing_pq",
                                  "nav_degree0", "nav_maxm33", "nav_map_short"])
def test_malformed_files_are_rejected(tmp_path, case):
    rng = np.random.default_rng(3)
    D = 8
    X = rng.integers(0, 256, (40, D)).astype(np.uint8)
    adj = [[(u + 1) % 40] for u in range(40)]
    nav = (list(range(0, 40, 4)), [[(i + 1) % 10] for i in range(10)], 0)
    idx, pqp, navd = write_custom_index(str(tmp_path), X, adj, 0, 2, nav=nav)
    piv = np.zeros((256, D), np.float32)
    cen = np.zeros((D, 1), np.float32)
    off = np.arange(D + 1, dtype=np.int32).reshape(-1, 1)
    if case == "nr3":
        _write_pivots_file(pqp + "_pivots.bin", [piv, cen, off], 3)
    elif case == "pivots255":
        _write_pivots_file(pqp + "_pivots.bin", [piv[:255], cen, off], 4)
    elif case == "chunks_short":
        _write_pivots_file(pqp + "_pivots.bin", [piv, cen, off[:-1] * 0 + np.arange(D).reshape(-1, 1)], 4)
    elif case == "chunks_decreasing":
        bad = off.copy()
        bad[3, 0] = 1
        _write_pivots_file(pqp + "_pivots.bin", [piv, cen, bad], 4)
    elif case == "codes_mismatch":
        with open(pqp + "_compressed.bin", "wb") as f:
            f.write(struct.pack("<ii", 40, D - 1) + bytes(40 * (D - 1)))
    elif case == "index_truncated":
        sz = os.path.getsize(idx)
        with open(idx, "r+b") as f:
            f.truncate(sz - 4096)
    elif case == "missing_pq":
        os.remove(pqp + "_compressed.bin")
    elif case == "nav_degree0":
        raw = bytearray(open(os.path.join(navd, "nav_index"), "rb").read())
        raw[24:28] = struct.pack("<I", 0)
        open(os.path.join(navd, "nav_index"), "wb").write(bytes(raw))
    elif case == "nav_maxm33":
        raw = bytearray(open(os.path.join(navd, "nav_index"), "rb").read())
        raw[8:12] = struct.pack("<I", 33)
        open(os.path.join(navd, "nav_index"), "wb").write(bytes(raw))
    elif case == "nav_map_short":
        with open(os.path.join(navd, "map.txt"), "w") as f:
            f.write("0\n4\n")
    with pytest.raises(RuntimeError):
        gi.inspect(idx, pqp, navd)


def test_vecs_roundtrip(tmp_path):
    rng = np.random.default_rng(4)
    for dt, ext in ((np.uint8, "bvecs"), (np.float32, "fvecs"), (np.int32, "ivecs")):
        A = (rng.integers(0, 200, (37, 13))).astype(dt)
        p = str(tmp_path / f"a.{ext}")
        gi.write_vecs(p, A)
        assert np.array_equal(gi.read_vecs(p, dt), A)
        assert os.path.getsize(p) == 37 * (4 + 13 * np.dtype(dt).itemsize)


def test_pivot_sampler_matches_gen_small_file_rule():
    # bin/gen_small_file.cpp:18-25: mt19937(114514) shuffle of 0..n-1, first
    # num_samp, sorted.  std::shuffle is libstdc++'s; check the invariants
    # and determinism.
    a = gi.sample_ids(10000, 500)
    b = gi.sample_ids(10000, 500)
    assert np.array_equal(a, b) and np.all(np.diff(a) > 0) and a.min() >= 0 and a.max() < 10000


@pytest.mark.parametrize("dtype,dim,M", [("uint8", 8, 2), ("uint8", 10, 3), ("float", 6, 4)])
def test_pq_encoder_rule(dtype, dim, M):
    # the host encoder's code = first argmin over the 256 pivots of
    # fma-accumulated ((x - centroid) - pivot)^2 in dim order, restated with
    # exact float32 rounding; the GPU encoder (gann_pq_encode) is checked
    # against the host encoder in tests/test_gpu_build.py
    from _helpers import fma_f32
    r = np.random.default_rng(dim)
    X = (r.integers(0, 256, (40, dim), dtype=np.uint8) if dtype == "uint8"
         else r.standard_normal((40, dim)).astype(np.float32))
    pq = gi.train_pq(X, M, sample=40, iters=3, seed=1)
    # a pivot equal to another makes the first one win
    piv, cen, off = pq.pivots, pq.centroid, pq.chunk_offsets
    for i in range(X.shape[0]):
        for m in range(M):
            lo, hi = int(off[m]), int(off[m + 1])
            best, bk = np.float32(np.inf), 0
            for k in range(256):
                d = np.float32(0.0)
                for j in range(lo, hi):
                    x = np.float32(np.float32(X[i, j]) - cen[j])
                    t = np.float32(x - piv[k, j])
                    d = fma_f32(t, t, d)
                if d < best:
                    best, bk = d, k
            assert pq.codes[i, m] == bk, (i, m)
