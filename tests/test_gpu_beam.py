"""GPU beam search (beam width 2..4, a mode of this library with no
counterpart in the reference) against the oracle's restatement of the same
mode (orc_search_beam, pinned to the reference search at width 1 by
tests/test_oracle_beam.py): ids, distances (bitwise), fill counts and
expansion counts must be identical on every query."""
import numpy as np
import pytest

import oracle as orc
from gustann_amd import FLOAT, MODE_FUSED, MODE_FUSED_GP, MODE_STEPWISE, UINT8, GannError, GustANN, GustANNConfig
from gustann_amd import index as gi

pytestmark = pytest.mark.gpu


def _open(meta, dtype):
    P = meta["paths"]
    g = GustANN(dtype)
    g.init_pure_mem(GustANNConfig(P["index"], P["pq"], P["nav"]), True)
    ix = orc.Index(P["index"], P["pq"], P["nav"], dtype="uint8" if dtype == UINT8 else "float")
    return g, ix


def _check(g, ix, Q, topk, L, bw, mode=MODE_FUSED):
    ne = np.empty(Q.shape[0], np.int32)
    nns, d, f = g.search(Q, Q.shape[0], topk, L, beam_width=bw, n_exp=ne, mode=mode)
    on, od, of, oe = ix.search_beam(Q, topk, L, bw, threads=8)
    assert np.array_equal(f, of)
    assert np.array_equal(nns, on)
    assert np.array_equal(d.view(np.uint32), od.view(np.uint32))
    assert np.array_equal(ne, oe)
    return nns


@pytest.fixture(scope="module")
def u8(tiny_u8):
    g, ix = _open(tiny_u8, UINT8)
    yield tiny_u8, g, ix
    g.close()


@pytest.mark.parametrize("bw", [2, 3, 4])
@pytest.mark.parametrize("L", [10, 40, 100])
def test_beam_u8(u8, bw, L):
    meta, g, ix = u8
    Q = gi.read_vecs(meta["paths"]["query"], np.uint8).astype(np.float32)
    _check(g, ix, Q, 10, L, bw)


@pytest.mark.parametrize("bw,L", [(2, 40), (4, 100), (4, 800)])
def test_beam_u8_pivots_through_caches(u8, bw, L):
    # the pivot table read from HBM instead of LDS (forced, and chosen by
    # GANN_MODE_FUSED itself at L = 800, where few lists fit beside the table)
    meta, g, ix = u8
    Q = gi.read_vecs(meta["paths"]["query"], np.uint8).astype(np.float32)
    _check(g, ix, Q, 10, L, bw, mode=MODE_FUSED_GP)
    if L == 800:
        _check(g, ix, Q, 10, L, bw)


def test_beam_topk100_lds_path(u8):
    # top-k above 64 keeps the top-k in LDS (C4 shape: top-100, L=200, width 4)
    meta, g, ix = u8
    Q = gi.read_vecs(meta["paths"]["query"], np.uint8).astype(np.float32)
    _check(g, ix, Q, 100, 200, 4)


@pytest.mark.parametrize("bw", [2, 4])
def test_beam_f32(tiny_f32, bw):
    g, ix = _open(tiny_f32, FLOAT)
    try:
        Q = gi.read_vecs(tiny_f32["paths"]["query"], np.float32)
        _check(g, ix, Q, 10, 64, bw)
    finally:
        g.close()


def test_beam_recall_close_to_width_one(u8):
    meta, g, ix = u8
    Q = gi.read_vecs(meta["paths"]["query"], np.uint8).astype(np.float32)
    gt = gi.read_vecs(meta["paths"]["gt"], np.int32)
    r1 = orc.recall(g.search(Q, Q.shape[0], 10, 40)[0], gt, 10)
    r4 = orc.recall(g.search(Q, Q.shape[0], 10, 40, beam_width=4)[0], gt, 10)
    assert r4 >= r1 - 0.05


def test_beam_limits(u8):
    meta, g, ix = u8
    Q = gi.read_vecs(meta["paths"]["query"], np.uint8).astype(np.float32)[:4]
    with pytest.raises(GannError):
        g.search(Q, 4, 10, 40, beam_width=5)
    with pytest.raises(GannError):
        g.search(Q, 4, 10, 40, beam_width=0)
    with pytest.raises(GannError):
        g.search(Q, 4, 10, 40, beam_width=2, mode=MODE_STEPWISE)
    nns, _, f = g.search(Q, 4, 10, 40, beam_width=2, mode=MODE_FUSED)
    assert (f == 10).all()


@pytest.mark.parametrize("bw", [1, 2, 4])
@pytest.mark.parametrize("mode", [MODE_FUSED, MODE_FUSED_GP])
def test_beam_known_answers(tmp_path, bw, mode):
    # the hand-worked traces of tests/_helpers.py (BEAM_EXPECT) on the kernel
    from _helpers import BEAM_EXPECT, write_beam_known_answer_index
    paths = write_beam_known_answer_index(str(tmp_path))
    g = GustANN(UINT8)
    g.init_pure_mem(GustANNConfig(paths[0], paths[1], ""), True)
    q = np.zeros((1, 4), np.float32)
    nexp, ids, dists = BEAM_EXPECT[bw]
    ne = np.empty(1, np.int32)
    nns, d, f = g.search(q, 1, 3, 4, beam_width=bw, n_exp=ne, mode=mode)
    g.close()
    assert ne[0] == nexp and f[0] == 3
    assert nns[0].tolist() == ids and d[0].tolist() == dists
