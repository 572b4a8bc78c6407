"""GPU parity against the CPU oracle on index shapes beyond one lane per
neighbour and beyond the register rerank: graph degree R up to 128 (the
reference's own index recipe, scripts/build_diskann_index.sh:7, builds
R = 128; its kernel runs roundup32(R) threads per query,
src/pure_mem.cu:137) and vectors of 384 and 512 dims (the reference's
square_sum_32 takes any dim, src/impl/util.cuh:26-46).  Every execution mode
and the beam search must return the oracle's ids, distance bits, fill counts
and expansion counts."""
import numpy as np
import pytest
from _helpers import write_custom_index
from test_search_semantics import random_graph

import oracle as orc
from gustann_amd import (FLOAT, MODE_FUSED, MODE_FUSED_GP, MODE_FUSED_LUT, MODE_STEPWISE, MODE_STEPWISE_PAGED,
                         UINT8, GustANN, GustANNConfig)
from gustann_amd import index as gi

pytestmark = pytest.mark.gpu

MODES = (MODE_FUSED, MODE_FUSED_LUT, MODE_FUSED_GP, MODE_STEPWISE, MODE_STEPWISE_PAGED)


def _open(paths, dtype):
    g = GustANN(dtype)
    g.init_pure_mem(GustANNConfig(*paths), True)
    return g


def _same(got, ref, ne, oe):
    nns, d, f = got
    on, od, of = ref
    assert np.array_equal(f, of)
    assert np.array_equal(nns, on)
    assert np.array_equal(np.ascontiguousarray(d).view(np.uint32), np.ascontiguousarray(od).view(np.uint32))
    assert np.array_equal(ne, oe)


def _check_all_modes(g, ix, Q, cases, beam_widths=(2, 4)):
    nq = Q.shape[0]
    for L, topk in cases:
        on, od, of, oe, _ = ix.search(Q, topk, L, threads=8)
        for mode in MODES:
            ne = np.empty(nq, np.int32)
            got = g.search(Q, nq, topk, L, n_exp=ne, mode=mode)
            _same(got, (on, od, of), ne, oe)
        for bw in beam_widths:
            bn, bd, bf, be = ix.search_beam(Q, topk, L, bw, threads=8)
            ne = np.empty(nq, np.int32)
            got = g.search(Q, nq, topk, L, beam_width=bw, n_exp=ne)
            _same(got, (bn, bd, bf), ne, be)


@pytest.mark.parametrize("R,D,M", [(96, 32, 16), (128, 32, 8), (128, 128, 32), (100, 64, 64)])
def test_degree_above_64_random_graphs(tmp_path, R, D, M):
    # degrees uniform in [1, R]: expansions with one and with two 64-neighbour
    # blocks; PQ shapes with the unrolled (M = 16, 32, 64) and generic (M = 8)
    # code paths
    rng = np.random.default_rng(R + D + M)
    n = 400
    X = rng.integers(0, 256, (n, D)).astype(np.uint8)
    adj = random_graph(rng, n, R)
    assert max(len(a) for a in adj) > 64
    pq = gi.train_pq(X, M, sample=n, iters=4, seed=R)
    paths = write_custom_index(str(tmp_path), X, adj, int(rng.integers(0, n)), R, pq=pq)
    g = _open(paths, UINT8)
    assert g.info.max_m == R
    ix = orc.Index(*paths[:2])
    Q = rng.integers(0, 256, (30, D)).astype(np.float32)
    _check_all_modes(g, ix, Q, [(16, 5), (64, 10), (300, 10), (200, 100)])
    g.close()


@pytest.fixture(scope="module")
def vamana_r128(tmp_path_factory):
    """A host-built Vamana graph with R = 128 (the reference's index recipe)
    over a 6k x 128 uint8 mixture, PQ M = 32, and a pivot graph."""
    spec = gi.DatasetSpec(name="r128", n=6000, dim=128, nclusters=30, R=128, L_build=160, M=32, nq=60, k=10,
                          nav_n=600, pq_sample=6000, pq_iters=6, alpha=1.2)
    return gi.build_dataset(spec, str(tmp_path_factory.mktemp("r128")))


def test_vamana_r128_index(vamana_r128):
    P = vamana_r128["paths"]
    g = _open((P["index"], P["pq"], P["nav"]), UINT8)
    ix = orc.Index(P["index"], P["pq"], P["nav"])
    assert g.info.max_m == 128 and g.info.node_len == 128 + 4 + 4 * 128
    Q = gi.read_vecs(P["query"], np.uint8).astype(np.float32)
    _check_all_modes(g, ix, Q, [(64, 10), (400, 10)], beam_widths=(4,))
    # the index really has expansions with more than 64 neighbours
    npp, nl = int(g.info.nodes_per_page), int(g.info.node_len)
    degs = [int(ix.pages[(u // npp) * 4096 + (u % npp) * nl + 128:][:4].view(np.int32)[0])
            for u in range(0, 6000, 7)]
    assert max(degs) > 64
    g.close()


def test_float_r128_c2_shape(tmp_path):
    # float D = 96, M = 48 (2-dim chunks), R = 128
    rng = np.random.default_rng(96)
    n, D, R = 400, 96, 128
    X = rng.standard_normal((n, D)).astype(np.float32)
    X /= np.linalg.norm(X, axis=1, keepdims=True)
    adj = random_graph(rng, n, R)
    pq = gi.train_pq(X, 48, sample=n, iters=4, seed=5)
    paths = write_custom_index(str(tmp_path), X, adj, 3, R, pq=pq)
    g = _open(paths, FLOAT)
    ix = orc.Index(*paths[:2], "", "float")
    Q = rng.standard_normal((30, D)).astype(np.float32)
    _check_all_modes(g, ix, Q, [(32, 10), (128, 10)])
    g.close()


@pytest.mark.parametrize("dtype,D,M,R", [("uint8", 384, 96, 64), ("float", 384, 48, 64), ("uint8", 384, 128, 96),
                                         ("float", 512, 64, 48)])
def test_dims_beyond_256(tmp_path, dtype, D, M, R):
    # 384 dims: 12 rerank coordinates per lane in registers; 512 dims: the
    # coordinates past 384 read from the record; the pivot-graph entry kernel
    # over the same vectors
    rng = np.random.default_rng(D + M + R)
    n = 300
    if dtype == "uint8":
        X = rng.integers(0, 256, (n, D)).astype(np.uint8)
        Q = rng.integers(0, 256, (24, D)).astype(np.float32)
    else:
        X = rng.standard_normal((n, D)).astype(np.float32)
        Q = rng.standard_normal((24, D)).astype(np.float32)
    adj = random_graph(rng, n, R)
    pq = gi.train_pq(X, M, sample=n, iters=3, seed=D)
    nav_ids = sorted(rng.choice(n, 40, replace=False).tolist())
    nav_adj = random_graph(rng, 40, 8)
    paths = write_custom_index(str(tmp_path), X, adj, int(rng.integers(0, n)), R, pq=pq,
                               nav=(nav_ids, nav_adj, 0))
    g = _open(paths, UINT8 if dtype == "uint8" else FLOAT)
    ix = orc.Index(*paths, dtype)
    ent, loc = g.nav_entry(Q)
    assert np.array_equal(loc, [ix.nav_entry_local(q)[0] for q in Q])
    assert np.array_equal(ent, [ix.entry(q)[0] for q in Q])
    _check_all_modes(g, ix, Q, [(24, 10), (96, 5)], beam_widths=(3,))
    g.close()
