"""GPU parity of entry selection and beam search against the CPU oracle.

The bar: uint8 exact distances bit-exact, ADC-driven trajectories identical,
so per-query result lists (ids, distances, fill counts, expansion counts) are
equal to the oracle's on every query -- stronger than the 99.5% top-k set
match and +-0.002 recall the reference comparison asks for.  Float indexes
are held to the same bar because the kernels reproduce the reference's
summation orders."""
import numpy as np
import pytest
from _helpers import exact_pq, write_custom_index
from test_search_semantics import random_graph

import oracle as orc
from gustann_amd import (FLOAT, MODE_FUSED, MODE_FUSED_GP, MODE_FUSED_LUT, MODE_STEPWISE, MODE_STEPWISE_PAGED,
                         MODE_STEPWISE_URING, UINT8,
                         GannError, GustANN,
                         GustANNConfig, GustANNStats)
from gustann_amd import index as gi

pytestmark = pytest.mark.gpu


def _open(paths, dtype=UINT8, nav=True, pinned=False):
    g = GustANN(dtype)
    g.init_pure_mem(GustANNConfig(paths[0], paths[1], paths[2] if nav else ""), not pinned)
    return g


def _paths(meta):
    P = meta["paths"]
    return P["index"], P["pq"], P["nav"]


def _queries(meta, dtype=np.uint8):
    return gi.read_vecs(meta["paths"]["query"], dtype).astype(np.float32)


def _assert_same(got, ref, nexp=None, rexp=None):
    nns, d, f = got
    on, od, of = ref
    assert np.array_equal(f, of)
    assert np.array_equal(nns, on)
    assert np.array_equal(np.ascontiguousarray(d).view(np.uint32), np.ascontiguousarray(od).view(np.uint32))
    if nexp is not None:
        assert np.array_equal(nexp, rexp)


@pytest.fixture(scope="module")
def u8(tiny_u8):
    g = _open(_paths(tiny_u8))
    ix = orc.Index(*_paths(tiny_u8))
    yield tiny_u8, g, ix
    g.close()


def test_nav_entries_match_oracle(u8):
    meta, g, ix = u8
    Q = _queries(meta)
    ent, loc = g.nav_entry(Q)
    assert np.array_equal(loc, [ix.nav_entry_local(q)[0] for q in Q])
    assert np.array_equal(ent, [ix.entry(q)[0] for q in Q])


@pytest.mark.parametrize("mode", [MODE_FUSED, MODE_FUSED_LUT, MODE_FUSED_GP])
@pytest.mark.parametrize("L,topk", [(10, 10), (16, 10), (40, 10), (100, 10), (64, 1), (200, 100),
                                    (700, 10)])
def test_fused_search_matches_oracle_u8(u8, L, topk, mode):
    meta, g, ix = u8
    Q = _queries(meta)
    ne = np.empty(Q.shape[0], np.int32)
    st = GustANNStats()
    got = g.search(Q, Q.shape[0], topk, L, n_exp=ne, stats=st, mode=mode)
    on, od, of, oe, _ = ix.search(Q, topk, L, threads=8)
    _assert_same(got, (on, od, of), ne, oe)
    assert st.n_expansions == int(oe.sum()) and st.n_nav_fallback == 0 and st.run_time > 0
    if topk == 10:
        gt = gi.read_vecs(meta["paths"]["gt"], np.int32)
        assert orc.recall(got[0], gt, 10) == orc.recall(on, gt, 10)


def test_stepwise_matches_fused_and_oracle(u8):
    meta, g, ix = u8
    Q = _queries(meta)[:120]
    ne = np.empty(Q.shape[0], np.int32)
    got = g.search(Q, Q.shape[0], 10, 32, mode=MODE_STEPWISE, n_exp=ne)
    on, od, of, oe, _ = ix.search(Q, 10, 32, threads=8)
    _assert_same(got, (on, od, of), ne, oe)


@pytest.mark.parametrize("pinned,mode", [(False, MODE_STEPWISE_PAGED), (True, MODE_STEPWISE_PAGED),
                                         (False, MODE_STEPWISE_URING)])
def test_paged_stepwise_matches_oracle(tiny_u8, pinned, mode):
    # pages come from the index file (pread of the record, or whole pages
    # through io_uring) or the pinned host image
    g = _open(_paths(tiny_u8), pinned=pinned)
    ix = orc.Index(*_paths(tiny_u8))
    Q = _queries(tiny_u8)[:120]
    ne = np.empty(Q.shape[0], np.int32)
    got = g.search(Q, Q.shape[0], 10, 32, mode=mode, n_exp=ne)
    on, od, of, oe, _ = ix.search(Q, 10, 32, threads=8)
    _assert_same(got, (on, od, of), ne, oe)
    g.close()


def test_medoid_entry_without_nav(tiny_u8):
    g = _open(_paths(tiny_u8), nav=False)
    ix = orc.Index(*_paths(tiny_u8)[:2])
    Q = _queries(tiny_u8)
    ent, loc = g.nav_entry(Q)
    assert np.all(ent == ix.medoid) and np.all(loc == -1)
    got = g.search(Q, Q.shape[0], 10, 48)
    on, od, of, _, _ = ix.search(Q, 10, 48, threads=8)
    _assert_same(got, (on, od, of))
    g.close()


def test_host_pinned_placement_matches(tiny_u8):
    g = _open(_paths(tiny_u8), pinned=True)
    ix = orc.Index(*_paths(tiny_u8))
    Q = _queries(tiny_u8)[:100]
    got = g.search(Q, Q.shape[0], 10, 40)
    on, od, of, _, _ = ix.search(Q, 10, 40, threads=8)
    _assert_same(got, (on, od, of))
    g.close()


@pytest.mark.parametrize("L", [16, 32, 64])
def test_fused_search_matches_oracle_float(tiny_f32, L):
    g = _open(_paths(tiny_f32), dtype=FLOAT)
    ix = orc.Index(*_paths(tiny_f32), dtype="float")
    Q = _queries(tiny_f32, np.float32)
    ent, loc = g.nav_entry(Q)
    assert np.array_equal(loc, [ix.nav_entry_local(q)[0] for q in Q])
    ne = np.empty(Q.shape[0], np.int32)
    got = g.search(Q, Q.shape[0], 10, L, n_exp=ne)
    on, od, of, oe, _ = ix.search(Q, 10, L, threads=8)
    _assert_same(got, (on, od, of), ne, oe)
    got2 = g.search(Q, Q.shape[0], 10, L, mode=MODE_STEPWISE)
    _assert_same(got2, (on, od, of))
    got3 = g.search(Q, Q.shape[0], 10, L, mode=MODE_FUSED_LUT)
    _assert_same(got3, (on, od, of))
    got4 = g.search(Q, Q.shape[0], 10, L, mode=MODE_STEPWISE_PAGED)
    _assert_same(got4, (on, od, of))
    got5 = g.search(Q, Q.shape[0], 10, L, mode=MODE_FUSED_GP)
    _assert_same(got5, (on, od, of))
    got6 = g.search(Q, Q.shape[0], 10, L, mode=MODE_STEPWISE_URING)
    _assert_same(got6, (on, od, of))
    g.close()


@pytest.mark.parametrize("seed,R,L,topk,trained", [(0, 12, 4, 3, False), (2, 12, 16, 10, True),
                                                   (4, 16, 6, 6, False), (5, 10, 40, 20, True),
                                                   (6, 64, 8, 8, False)])
def test_random_graphs_match_oracle(tmp_path, seed, R, L, topk, trained):
    rng = np.random.default_rng(seed)
    n, D = 300, 16
    X = rng.integers(0, 256, (n, D)).astype(np.uint8)
    adj = random_graph(rng, n, R)
    pq = gi.train_pq(X, 4, sample=n, iters=4, seed=seed) if trained else exact_pq(X)
    paths = write_custom_index(str(tmp_path), X, adj, int(rng.integers(0, n)), R, pq=pq)
    g = _open(paths, nav=False)
    ix = orc.Index(*paths[:2])
    Q = rng.integers(0, 256, (40, D)).astype(np.float32)
    on, od, of, oe, _ = ix.search(Q, topk, L)
    for mode in (MODE_FUSED, MODE_FUSED_LUT, MODE_FUSED_GP, MODE_STEPWISE, MODE_STEPWISE_PAGED, MODE_STEPWISE_URING):
        ne = np.empty(40, np.int32)
        got = g.search(Q, 40, topk, L, n_exp=ne, mode=mode)
        _assert_same(got, (on, od, of), ne, oe)
    g.close()


def test_complete_graph_known_answer(tmp_path):
    n, D = 20, 8
    X = np.zeros((n, D), np.uint8)
    X[:, 0] = np.arange(n) * 3
    adj = [[v for v in range(n) if v != u] for u in range(n)]
    paths = write_custom_index(str(tmp_path), X, adj, 5, 24)
    g = _open(paths, nav=False)
    q = np.zeros((1, D), np.float32)
    q[0, 0] = 7.0
    ne = np.empty(1, np.int32)
    nns, d, f = g.search(q, 1, 10, 32, n_exp=ne)
    d_all = sorted([(float((7 - 3 * i) ** 2), i) for i in range(n)] + [(64.0, 5)])
    assert ne[0] == n + 1 and f[0] == 10
    assert list(nns[0]) == [i for _, i in d_all[:10]] and list(d[0]) == [x for x, _ in d_all[:10]]
    g.close()


def test_nav_known_answers(tmp_path):
    D = 32
    X = np.full((4, D), 100, np.uint8)
    X[0, 2], X[1, 0], X[2, 0], X[3, 1] = 110, 106, 105, 105
    base_adj = [[(u + 1) % 4] for u in range(4)]
    paths = write_custom_index(str(tmp_path / "tie"), X, base_adj, 0, 4,
                               nav=([0, 1, 2, 3], [[1, 2, 3], [0], [0], [0]], 0))
    g = _open(paths)
    ent, loc = g.nav_entry(np.full((1, D), 100, np.float32))
    assert loc[0] == 3 and ent[0] == 3
    g.close()
    X2 = np.full((2, 16), 50, np.uint8)
    X2[1, 0] = 52
    paths = write_custom_index(str(tmp_path / "deg"), X2, [[1], [0]], 1, 2, nav=([0, 1], [[1], [0]], 0))
    g = _open(paths)
    q = np.full((3, 16), 50, np.float32)
    q[:, 0] = 53.0
    ent, loc = g.nav_entry(q)
    assert np.all(loc == 0x7FFFFFFF) and np.all(ent == 1)  # fallback to the medoid
    st = GustANNStats()
    g.search(q, 3, 1, 2, stats=st)
    assert st.n_nav_fallback == 3
    g.close()


def test_replicated_queries_give_identical_rows(u8):
    # search_mem replicates the query set -R times (bin/search_disk.cpp:172-183).
    meta, g, _ = u8
    Q = _queries(meta)[:50]
    nns, d, f = g.search(np.tile(Q, (4, 1)), 200, 10, 32)
    for r in range(1, 4):
        assert np.array_equal(nns[:50], nns[50 * r:50 * (r + 1)])


def test_argument_errors(u8):
    meta, g, _ = u8
    Q = _queries(meta)[:4]
    with pytest.raises(GannError) as e:
        g.search(Q, 4, 10, 5)  # L < topk
    assert e.value.code == 1
    with pytest.raises(GannError) as e:
        g.search(Q, 4, 10, 20, beam_width=5)  # widths 2..4 are the beam search mode
    assert e.value.code == 6
    nns, d, f = g.search(Q[:0], 0, 10, 20)
    assert nns.shape == (0, 10)


def test_search_device_matches_host_api(u8):
    import torch
    meta, g, _ = u8
    Q = _queries(meta)
    nq = Q.shape[0]
    dev = torch.device("cuda:0")
    q_t = torch.from_numpy(Q).to(dev)
    ent = torch.empty(nq, dtype=torch.int32, device=dev)
    nns = torch.empty((nq, 10), dtype=torch.int32, device=dev)
    dd = torch.empty((nq, 10), dtype=torch.float32, device=dev)
    fc = torch.empty(nq, dtype=torch.int32, device=dev)
    s = torch.cuda.Stream()
    g.search_device(q_t.data_ptr(), nq, 10, 48, ent.data_ptr(), nns.data_ptr(), dd.data_ptr(),
                    fc.data_ptr(), stream=s.cuda_stream)
    s.synchronize()
    hn, hd, hf = g.search(Q, nq, 10, 48)
    assert np.array_equal(nns.cpu().numpy(), hn) and np.array_equal(fc.cpu().numpy(), hf)
    assert np.array_equal(dd.cpu().numpy().view(np.uint32), hd.view(np.uint32))


@pytest.mark.parametrize("seed", [11, 12])
def test_zero_degree_nodes_match_oracle(tmp_path, seed):
    # records with degree 0 (including, for seed 12, possibly the entry):
    # every mode, and the beam search, must agree with the oracle
    rng = np.random.default_rng(seed)
    n, D, R = 200, 16, 10
    X = rng.integers(0, 256, (n, D)).astype(np.uint8)
    adj = random_graph(rng, n, R, min_deg=0)
    for u in rng.choice(n, 30, replace=False):
        adj[int(u)] = []
    medoid = int(rng.integers(0, n))
    if seed == 12:
        adj[medoid] = []
    paths = write_custom_index(str(tmp_path), X, adj, medoid, R)
    g = _open(paths, nav=False)
    ix = orc.Index(*paths[:2])
    Q = rng.integers(0, 256, (30, D)).astype(np.float32)
    on, od, of, oe, _ = ix.search(Q, 5, 12)
    for mode in (MODE_FUSED, MODE_FUSED_LUT, MODE_FUSED_GP, MODE_STEPWISE, MODE_STEPWISE_PAGED, MODE_STEPWISE_URING):
        ne = np.empty(30, np.int32)
        got = g.search(Q, 30, 5, 12, n_exp=ne, mode=mode)
        _assert_same(got, (on, od, of), ne, oe)
    bn, bd, bf, be = ix.search_beam(Q, 5, 12, 3)
    ne = np.empty(30, np.int32)
    got = g.search(Q, 30, 5, 12, beam_width=3, n_exp=ne)
    _assert_same(got, (bn, bd, bf), ne, be)
    g.close()


@pytest.mark.parametrize("form", ["split", "half", "cache", "wide"])
def test_pivot_table_forms_match_oracle(u8, form, monkeypatch):
    # all but the last group of 8 chunks of the pivot table in LDS ("split"),
    # its first half ("half"), or the whole table read through the caches
    # ("cache"), with all 32 pivot rows of a lookup requested at once in
    # 8-wave workgroups ("wide"); GANN_PIVOT_FORM forces the form at every L
    meta, g, ix = u8
    Q = _queries(meta)
    monkeypatch.setenv("GANN_PIVOT_FORM", form)
    for L, topk in ((40, 10), (300, 10), (200, 100)):
        ne = np.empty(Q.shape[0], np.int32)
        got = g.search(Q, Q.shape[0], topk, L, n_exp=ne)
        on, od, of, oe, _ = ix.search(Q, topk, L, threads=8)
        _assert_same(got, (on, od, of), ne, oe)


@pytest.mark.parametrize("mode,bw", [(MODE_FUSED, 1), (MODE_FUSED_GP, 1), (MODE_FUSED, 3)])
def test_query_order_changes_no_result(u8, monkeypatch, mode, bw):
    # with a pivot graph the fused kernels take the queries farthest from
    # their entry first (GANN_QUERY_ORDER=0: in queue order); every output
    # stays the same and equal to the oracle's (beam width 1)
    meta, g, ix = u8
    Q = _queries(meta)
    Q = np.concatenate([Q, Q[::-1], Q[::2]])
    runs = []
    for env in ("1", "0"):
        monkeypatch.setenv("GANN_QUERY_ORDER", env)
        ne = np.empty(Q.shape[0], np.int32)
        got = g.search(Q, Q.shape[0], 10, 64, beam_width=bw, mode=mode, n_exp=ne)
        runs.append((got, ne))
    _assert_same(runs[0][0], runs[1][0], runs[0][1], runs[1][1])
    if bw == 1:
        on, od, of, oe, _ = ix.search(Q, 10, 64, threads=8)
        _assert_same(runs[0][0], (on, od, of), runs[0][1], oe)


@pytest.mark.parametrize("dtype,D,M,R", [("uint8", 32, 16, 64), ("uint8", 64, 16, 40), ("uint8", 64, 32, 64),
                                         ("float", 96, 48, 64), ("uint8", 128, 64, 48), ("uint8", 128, 32, 100)])
def test_wide_lookup_form_matches_oracle(tmp_path, monkeypatch, dtype, D, M, R):
    # the wide lookup form on each shape it serves (16 to 64 chunks of 2 or
    # 4 dims, at most 128 dims), one or two neighbour blocks, ragged degrees
    # down to 0 and a full-degree entry node, against the oracle
    rng = np.random.default_rng(D * 7 + M + R)
    n = 600
    if dtype == "uint8":
        X = rng.integers(0, 256, (n, D)).astype(np.uint8)
        Q = rng.integers(0, 256, (48, D)).astype(np.float32)
    else:
        X = rng.standard_normal((n, D)).astype(np.float32)
        Q = rng.standard_normal((48, D)).astype(np.float32)
    adj = random_graph(rng, n, R, min_deg=0)
    adj[1] = [int(v) for v in rng.choice(np.arange(2, n), size=R, replace=False)]
    pq = gi.train_pq(X, M, sample=n, iters=4, seed=D + M)
    paths = write_custom_index(str(tmp_path), X, adj, 1, R, pq=pq)
    g = _open(paths, dtype=UINT8 if dtype == "uint8" else FLOAT, nav=False)
    ix = orc.Index(*paths[:2], "", dtype)
    monkeypatch.setenv("GANN_PIVOT_FORM", "wide")
    for L, topk in ((12, 5), (64, 10), (300, 100)):
        on, od, of, oe, _ = ix.search(Q, topk, L)
        # the first 0, 1 or 3 chunks from a partial pivot table in LDS (one
        # neighbour block; with two the form keeps none)
        for wl in ("0", "1", "3"):
            monkeypatch.setenv("GANN_WIDE_LDS", wl)
            ne = np.empty(48, np.int32)
            got = g.search(Q, 48, topk, L, n_exp=ne, mode=MODE_FUSED)
            _assert_same(got, (on, od, of), ne, oe)
    monkeypatch.delenv("GANN_WIDE_LDS", raising=False)
    monkeypatch.delenv("GANN_PIVOT_FORM", raising=False)
    g.close()


@pytest.mark.parametrize("dtype,D,M", [("uint8", 192, 48), ("uint8", 256, 64), ("float", 192, 48)])
def test_wide_vectors_match_oracle(tmp_path, monkeypatch, dtype, D, M):
    # dim > 128: the kernels that keep 8 rerank coordinates per lane (4-dim
    # PQ chunks, so the unrolled ADC path); every fused form of the pivot
    # table, the per-query LUT kernel and the beam search
    rng = np.random.default_rng(D + M)
    n, R = 300, 16
    if dtype == "uint8":
        X = rng.integers(0, 256, (n, D)).astype(np.uint8)
        Q = rng.integers(0, 256, (40, D)).astype(np.float32)
    else:
        X = rng.standard_normal((n, D)).astype(np.float32)
        Q = rng.standard_normal((40, D)).astype(np.float32)
    adj = random_graph(rng, n, R)
    pq = gi.train_pq(X, M, sample=n, iters=4, seed=D)
    paths = write_custom_index(str(tmp_path), X, adj, int(rng.integers(0, n)), R, pq=pq)
    g = _open(paths, dtype=UINT8 if dtype == "uint8" else FLOAT, nav=False)
    ix = orc.Index(*paths[:2], "", dtype)
    for L, topk in ((24, 10), (96, 5)):
        on, od, of, oe, _ = ix.search(Q, topk, L)
        runs = [(None, MODE_FUSED), (None, MODE_FUSED_LUT), (None, MODE_FUSED_GP),
                ("half", MODE_FUSED), ("cache", MODE_FUSED)]
        for form, mode in runs:
            if form is None:
                monkeypatch.delenv("GANN_PIVOT_FORM", raising=False)
            else:
                monkeypatch.setenv("GANN_PIVOT_FORM", form)
            ne = np.empty(40, np.int32)
            got = g.search(Q, 40, topk, L, n_exp=ne, mode=mode)
            _assert_same(got, (on, od, of), ne, oe)
        monkeypatch.delenv("GANN_PIVOT_FORM", raising=False)
        bn, bd, bf, be = ix.search_beam(Q, topk, L, 4)
        ne = np.empty(40, np.int32)
        got = g.search(Q, 40, topk, L, beam_width=4, n_exp=ne)
        _assert_same(got, (bn, bd, bf), ne, be)
    g.close()
