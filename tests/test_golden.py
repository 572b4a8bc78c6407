"""The committed golden fixtures (tests/golden/, written by make_golden.py):
the oracle must still reproduce them bit for bit, and their values are pinned
independently of the oracle -- exact integer L2 for uint8 results, float64
closed forms for the LUT, ADC and float distances, the pivot map for entries,
list order and fill rules for the search outputs."""
import json
import os

import numpy as np
import pytest

import oracle as orc
from gustann_amd import index as gi

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NAMES = ["u8_small", "f32_small"]


def load(name):
    d = os.path.join(GOLDEN, name)
    with open(os.path.join(d, "golden.json")) as f:
        spec = json.load(f)
    files = {k: os.path.join(d, v) for k, v in spec["files"].items()}
    exp = dict(np.load(os.path.join(d, "expected.npz")))
    qdt = np.uint8 if spec["dtype"] == "uint8" else np.float32
    Q = gi.read_vecs(files["query"], qdt).astype(np.float32)
    return spec, files, exp, Q


def base_vectors(index_file, dtype):
    """Every record's coordinates, read straight from the disk-index pages
    (record u at 4096 + (u / npp) * 4096 + (u % npp) * node_len,
    src/pure_mem.cuh:261-265)."""
    hdr = np.fromfile(index_file, np.uint64, count=9, offset=8)
    n, dim, _, node_len, npp = (int(v) for v in hdr[:5])
    es = 1 if dtype == "uint8" else 4
    raw = np.fromfile(index_file, np.uint8, offset=4096)
    u = np.arange(n)
    starts = (u // npp) * 4096 + (u % npp) * node_len
    rows = raw[starts[:, None] + np.arange(dim * es)[None, :]]
    return rows.view(np.uint8 if es == 1 else np.float32).reshape(n, dim)


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_golden(name):
    spec, files, exp, Q = load(name)
    ix = orc.Index(files["index"], files["pq"], files["nav"], spec["dtype"])
    assert (ix.num_pts, ix.dim, ix.medoid) == (spec["num_pts"], spec["dim"], spec["medoid"])
    for i in range(spec["nlut"]):
        lut = orc.lut_build(ix.pivots, ix.centroid, ix.chunk_offsets, Q[i])
        assert np.array_equal(lut.view(np.uint32), exp["lut"][i].view(np.uint32))
    adc = orc.adc_scan(ix.pivots, ix.centroid, ix.chunk_offsets, ix.codes, Q, exp["adc_ids"], 4)
    assert np.array_equal(adc.view(np.uint32), exp["adc"].view(np.uint32))
    assert [ix.nav_entry_local(q)[0] for q in Q] == exp["nav_local"].tolist()
    assert [ix.entry(q)[0] for q in Q] == exp["entry"].tolist()
    for L, k in spec["search_cases"]:
        nns, d, f, e, bad = ix.search(Q, k, L, threads=4, check=True)
        assert bad == 0
        assert np.array_equal(nns, exp[f"s{L}_{k}_nns"]) and np.array_equal(f, exp[f"s{L}_{k}_found"])
        assert np.array_equal(d.view(np.uint32), exp[f"s{L}_{k}_dists"].view(np.uint32))
        assert np.array_equal(e, exp[f"s{L}_{k}_nexp"])
    for w, L, k in spec["beam_cases"]:
        nns, d, f, e = ix.search_beam(Q, k, L, w, threads=4)
        p = f"b{w}_{L}_{k}_"
        assert np.array_equal(nns, exp[p + "nns"]) and np.array_equal(f, exp[p + "found"])
        assert np.array_equal(d.view(np.uint32), exp[p + "dists"].view(np.uint32))
        assert np.array_equal(e, exp[p + "nexp"])


@pytest.mark.parametrize("name", NAMES)
def test_golden_files_parse(name):
    spec, files, _, _ = load(name)
    info = gi.inspect(files["index"], files["pq"], files["nav"], 1 if spec["dtype"] == "uint8" else 4)
    assert info["num_pts"] == spec["num_pts"] and info["dim"] == spec["dim"]
    assert info["medoid"] == spec["medoid"] and info["pq_num_chunks"] == spec["num_chunks"]
    assert info["pq_num_pts"] == spec["num_pts"] and info["nav_num_node"] > 0


@pytest.mark.parametrize("name", NAMES)
def test_golden_lut_and_adc_closed_form(name):
    # LUT[m][c] = sum over the chunk's dims of (q_i - mu_i - P[c][i])^2 in
    # float64; ADC = sum over chunks of LUT[m][code_m]
    spec, files, exp, Q = load(name)
    pq = gi.read_pq(files["pq"])
    P = pq.pivots.astype(np.float64)
    mu = pq.centroid.astype(np.float64)
    off = pq.chunk_offsets
    M = off.shape[0] - 1
    for i in range(spec["nlut"]):
        r = (Q[i].astype(np.float64) - mu)[None, :] - P
        ref = np.stack([(r[:, off[m]:off[m + 1]] ** 2).sum(1) for m in range(M)])
        assert np.allclose(exp["lut"][i], ref, rtol=1e-5, atol=1e-5 * ref.max())
    ids = exp["adc_ids"]
    for qi in range(Q.shape[0]):
        r = (Q[qi].astype(np.float64) - mu)[None, :] - P
        lut = np.stack([(r[:, off[m]:off[m + 1]] ** 2).sum(1) for m in range(M)])
        codes = pq.codes[ids[qi]]
        ref = lut[np.arange(M)[None, :], codes].sum(1)
        assert np.allclose(exp["adc"][qi], ref, rtol=1e-5, atol=0)


@pytest.mark.parametrize("name", NAMES)
def test_golden_search_outputs_pinned(name):
    spec, files, exp, Q = load(name)
    X = base_vectors(files["index"], spec["dtype"])
    for tag, k in [(f"s{L}_{k}_", k) for L, k in spec["search_cases"]] + \
                  [(f"b{w}_{L}_{k}_", k) for w, L, k in spec["beam_cases"]]:
        nns, d, f = exp[tag + "nns"], exp[tag + "dists"], exp[tag + "found"]
        assert np.all((f >= 1) & (f <= k))
        for q in range(Q.shape[0]):
            ids, dd = nns[q, :f[q]], d[q, :f[q]]
            assert np.all(np.diff(dd) >= 0)  # retset_push_32 keeps the list sorted
            assert np.all((ids >= 0) & (ids < spec["num_pts"]))
            if spec["dtype"] == "uint8":
                # exact rerank: integer L2, exactly representable in f32
                ref = ((X[ids].astype(np.int64) - Q[q].astype(np.int64)) ** 2).sum(1)
                assert np.array_equal(dd.astype(np.int64), ref) and np.all(dd == ref.astype(np.float32))
            else:
                ref = ((X[ids].astype(np.float64) - Q[q].astype(np.float64)) ** 2).sum(1)
                assert np.allclose(dd, ref, rtol=1e-5, atol=1e-6)
    # the entry is the pivot-map image of the pivot-local nearest node
    mapping = np.loadtxt(os.path.join(files["nav"], "map.txt"), dtype=np.int64).reshape(-1)
    loc, ent = exp["nav_local"], exp["entry"]
    assert np.all((loc >= 0) & (loc < mapping.shape[0]))
    assert np.array_equal(ent, mapping[loc])
    # larger lists never lose recall on these fixtures' ground truth, and the
    # widest search finds nearly all true top-10
    gt = gi.read_vecs(files["gt"], np.int32)
    rec = [orc.recall(np.ascontiguousarray(exp[f"s{L}_{k}_nns"][:, :10]), gt, 10)
           for L, k in spec["search_cases"] if k >= 10]
    assert rec == sorted(rec) and rec[-1] >= 0.9
