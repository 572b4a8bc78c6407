"""check_recall (bin/check_recall.cpp behaviour) on hand-made files: the
recall value of calc_recall (bin/utils.hpp:104-116) and the two mismatch
errors."""
import os
import subprocess

import numpy as np
import pytest

from gustann_amd import index as gi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOOL = os.path.join(ROOT, "gustann_amd", "lib", "check_recall")


def _bin(path, a):
    a = np.asarray(a, dtype=np.int32)
    with open(path, "wb") as f:
        np.array(a.shape, dtype=np.int32).tofile(f)
        a.tofile(f)


def _run(*args):
    return subprocess.run([TOOL, *args], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                          text=True, timeout=30)


@pytest.fixture
def files(tmp_path):
    gt = np.array([[1, 2, 3, 4, 5], [10, 11, 12, 13, 14], [7, 8, 9, 6, 5]], dtype=np.int32)
    gpath = str(tmp_path / "gt.ivecs")
    gi.write_vecs(gpath, gt)
    return tmp_path, gpath


def test_recall_value(files):
    d, gpath = files
    res = str(d / "res.bin")
    # row 0: {2, 9} vs top-2 {1, 2} -> 1 hit; row 1: {11, 10} -> 2; row 2: {5, 6} vs {7, 8} -> 0
    _bin(res, [[2, 9], [11, 10], [5, 6]])
    r = _run(res, gpath)
    assert r.returncode == 0, r.stdout
    assert r.stdout.strip() == "Recall @ 2: 0.5"


def test_dim_mismatch(files):
    d, gpath = files
    res = str(d / "wide.bin")
    _bin(res, np.zeros((3, 6)))
    r = _run(res, gpath)
    assert r.returncode != 0 and "DIM mismatch: 5 vs 6" in r.stdout


def test_num_mismatch(files):
    d, gpath = files
    res = str(d / "short.bin")
    _bin(res, np.zeros((2, 2)))
    r = _run(res, gpath)
    assert r.returncode != 0 and "NUM mismatch: 3 vs 2" in r.stdout


def test_usage():
    r = _run("only_one_arg")
    assert r.returncode != 0 and "output_bin ground_truth_bin" in r.stdout
