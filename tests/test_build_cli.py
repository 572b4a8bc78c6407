"""build_disk_index command line (host builder): the files the reference's
DiskANN steps produce, readable by the search library's own readers, with a
pivot graph and exact ground truth; the oracle searches them."""
import os

import numpy as np
import pytest

import oracle as orc
from gustann_amd import build_disk_index as bdi
from gustann_amd import index as gi


def _write_bin(path, A):
    with open(path, "wb") as f:
        np.array(A.shape, np.int32).tofile(f)
        np.ascontiguousarray(A).tofile(f)


def test_build_from_bin_with_pivot_graph_and_gt(tmp_path):
    X, _ = gi.gen_mixture_u8(3000, 32, 20, 5, 6, threads=4)
    Qb, _ = gi.gen_mixture_u8(50, 32, 20, 5, 7, threads=4)
    _write_bin(str(tmp_path / "base.u8bin"), X)
    _write_bin(str(tmp_path / "q.u8bin"), Qb)
    pre = str(tmp_path / "idx")
    rc = bdi.main(["--data_type", "uint8", "--dist_fn", "l2", "--index_path_prefix", pre,
                   "--data_path", str(tmp_path / "base.u8bin"), "-R", "24", "-L", "40",
                   "-B", str(3000 * 8 / (1 << 30)), "--builder", "cpu",
                   "--pivot_graph", str(tmp_path / "nav"), "--pivot_samples", "300",
                   "--query_path", str(tmp_path / "q.u8bin"), "--gt_path", str(tmp_path / "gt.ivecs"),
                   "--gt_k", "10"])
    assert rc == 0
    info = gi.inspect(pre + "_disk.index", pre + "_pq", str(tmp_path / "nav"))
    assert info["num_pts"] == 3000 and info["dim"] == 32 and info["pq_num_chunks"] == 8
    assert info["nav_num_node"] == 300
    gt = gi.read_vecs(str(tmp_path / "gt.ivecs"), np.int32)
    ref, _ = gi.brute_force_knn(X, Qb.astype(np.float32), 10)
    assert np.array_equal(gt, ref)
    ix = orc.Index(pre + "_disk.index", pre + "_pq", str(tmp_path / "nav"))
    nns, _, _, _, _ = ix.search(Qb.astype(np.float32), 10, 64)
    assert orc.recall(nns, gt, 10) > 0.8


def test_build_from_fvecs_host(tmp_path):
    r = np.random.default_rng(3)
    X = r.standard_normal((1500, 24)).astype(np.float32)
    gi.write_vecs(str(tmp_path / "base.fvecs"), X)
    pre = str(tmp_path / "f")
    assert bdi.main(["--data_type", "float", "--index_path_prefix", pre, "--data_path",
                     str(tmp_path / "base.fvecs"), "-R", "16", "-L", "32", "--pq_chunks", "12",
                     "--builder", "cpu"]) == 0
    info = gi.inspect(pre + "_disk.index", pre + "_pq", "", elem_size=4)
    assert info["num_pts"] == 1500 and info["pq_num_chunks"] == 12


def test_bad_data_file(tmp_path):
    p = tmp_path / "bad.bin"
    np.array([10, 4], np.int32).tofile(str(p))
    with pytest.raises(ValueError):
        bdi.read_data(str(p), "uint8")
    assert bdi.pq_chunks_for_budget(1000, 128, 1000 * 16 / (1 << 30)) == 16
    assert bdi.pq_chunks_for_budget(1000, 8, 1.0) == 8
