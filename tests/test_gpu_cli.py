"""The search_mem command line (bin/search_disk.cpp flags and output lines)
over the C ABI: single-L run with the result preview and [REPORT] line, and
the L-sweep table; recall equals the oracle's on the same index."""
import os
import re
import subprocess

import numpy as np
import pytest

import oracle as orc
from gustann_amd import index as gi

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "gustann_amd", "lib", "search_mem")


def _run(args):
    r = subprocess.run([CLI, *args], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stdout
    return r.stdout


def test_single_L_reports_recall(tiny_u8):
    P = tiny_u8["paths"]
    out = _run(["--query", P["query"], "--index", P["index"], "--pq_data", P["pq"], "--nav_graph",
                P["nav"], "--data_type", "uint8", "--ground_truth", P["gt"], "--topk", "10",
                "--ef_search", "40", "-R", "2", "-G"])
    m = re.search(r"\[REPORT\] RECALL: ([0-9.]+)", out)
    assert m and "Recall @ 10:" in out
    ix = orc.Index(P["index"], P["pq"], P["nav"])
    Q = gi.read_vecs(P["query"], np.uint8).astype(np.float32)
    gt = gi.read_vecs(P["gt"], np.int32)
    nns, _, _, _, _ = ix.search(Q, 10, 40, threads=8)
    assert abs(float(m.group(1)) - orc.recall(nns, gt, 10)) < 1e-6
    preview = [l for l in out.splitlines() if "(" in l and "\t" in l]
    assert len(preview) == 5


@pytest.mark.parametrize("mode", ["fused", "gp", "lut", "stepwise", "paged", "uring"])
def test_sweep_table(tiny_u8, mode):
    P = tiny_u8["paths"]
    out = _run(["--query", P["query"], "--index", P["index"], "--pq_data", P["pq"], "--data_type",
                "uint8", "--ground_truth", P["gt"], "--topk", "10", "--ef_search", "10", "20", "40",
                "-R", "1", "-G", "--mode", mode])
    rows = [l.split() for l in out.splitlines()
            if re.match(r"^\d+\s+[0-9.]+\s+[0-9.]+\s+[0-9.]+$", l.strip())]
    assert [int(r[0]) for r in rows] == [10, 20, 40]
    recalls = [float(r[3]) for r in rows]
    assert recalls[0] <= recalls[1] + 0.02 <= recalls[2] + 0.04


def test_rejects_L_below_topk(tiny_u8):
    P = tiny_u8["paths"]
    r = subprocess.run([CLI, "--query", P["query"], "--index", P["index"], "--pq_data", P["pq"],
                        "--data_type", "uint8", "--topk", "10", "--ef_search", "5"],
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=60)
    assert r.returncode != 0 and "ef_search must be >= topk" in r.stdout


def test_result_file_and_check_recall(tiny_u8, tmp_path):
    P = tiny_u8["paths"]
    res = str(tmp_path / "res.bin")
    out = _run(["--query", P["query"], "--index", P["index"], "--pq_data", P["pq"], "--data_type",
                "uint8", "--ground_truth", P["gt"], "--topk", "10", "--ef_search", "40", "-R", "1",
                "-G", "--result_path", res])
    reported = float(re.search(r"\[REPORT\] RECALL: ([0-9.]+)", out).group(1))
    gt = gi.read_vecs(P["gt"], np.int32)
    ids = np.fromfile(res, dtype=np.int32)
    nq, k = int(ids[0]), int(ids[1])
    assert k == 10 and nq * k == ids.size - 2
    if gt.shape[0] != nq:  # check_recall needs one ground-truth row per result row
        return
    r = subprocess.run([os.path.join(ROOT, "gustann_amd", "lib", "check_recall"), res, P["gt"]],
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=60)
    assert r.returncode == 0, r.stdout
    m = re.search(r"Recall @ 10: ([0-9.e-]+)", r.stdout)
    assert m and abs(float(m.group(1)) - reported) < 1e-5


def test_beam_width_zipf_top100_sweep(tmp_path):
    # the Zipf configuration's shape through the command line: Zipf(1.1)
    # query clusters, top-100, L = 200 (and 256), beam width 4; the reported
    # recall is the oracle's beam search's
    spec = gi.DatasetSpec(name="zipf_cli", n=20_000, dim=128, nclusters=100, R=32, L_build=64, M=32, nq=120,
                          k=100, zipf_s=1.1, builder="gpu")
    P = gi.build_dataset(spec, str(tmp_path / "z"))["paths"]
    out = _run(["--query", P["query"], "--index", P["index"], "--pq_data", P["pq"], "--data_type", "uint8",
                "--ground_truth", P["gt"], "--topk", "100", "--ef_search", "200", "256", "-R", "1", "-G",
                "--beam_width", "4"])
    rows = [l.split() for l in out.splitlines()
            if re.match(r"^\d+\s+[0-9.]+\s+[0-9.]+\s+[0-9.]+$", l.strip())]
    assert [int(r[0]) for r in rows] == [200, 256]
    ix = orc.Index(P["index"], P["pq"], "")
    Q = gi.read_vecs(P["query"], np.uint8).astype(np.float32)
    gt = gi.read_vecs(P["gt"], np.int32)
    for row, L in zip(rows, (200, 256)):
        nns = ix.search_beam(Q, 100, L, 4, threads=8)[0]
        assert abs(float(row[3]) - orc.recall(nns, gt, 100)) < 1e-6


def test_rejects_beam_width_below_one(tiny_u8):
    P = tiny_u8["paths"]
    r = subprocess.run([CLI, "--query", P["query"], "--index", P["index"], "--pq_data", P["pq"],
                        "--data_type", "uint8", "--topk", "10", "--ef_search", "20", "--beam_width", "0"],
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=60)
    assert r.returncode != 0 and "--beam_width must be >= 1" in r.stdout
