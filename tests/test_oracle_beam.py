"""The oracle's beam search (orc_search_beam) against the reference
restatement: with beam width 1 it is the same algorithm as orc_search (the
reference's one node per iteration), so every output must be identical; with
wider beams it must reproduce the hand-worked traces of a 12-node graph
(expansion counts and top-k at widths 1, 2 and 4) and still return exact
distances in order and a recall close to width 1's."""
import numpy as np
import pytest

import oracle as orc
from gustann_amd import index as gi


@pytest.mark.parametrize("L", [10, 40, 100])
def test_beam1_is_reference_search(tiny_u8, L):
    P = tiny_u8["paths"]
    ix = orc.Index(P["index"], P["pq"], P["nav"])
    Q = gi.read_vecs(P["query"], np.uint8).astype(np.float32)[:120]
    a = ix.search(Q, 10, L, threads=8)
    b = ix.search_beam(Q, 10, L, 1, threads=8)
    assert np.array_equal(a[0], b[0])
    assert np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32))
    assert np.array_equal(a[2], b[2]) and np.array_equal(a[3], b[3])


@pytest.mark.parametrize("bw", [2, 4])
def test_wider_beam_exact_and_sorted(tiny_u8, bw):
    P = tiny_u8["paths"]
    ix = orc.Index(P["index"], P["pq"], P["nav"])
    Q = gi.read_vecs(P["query"], np.uint8).astype(np.float32)[:120]
    gt = gi.read_vecs(P["gt"], np.int32)[:120]
    nns, d, found, nexp = ix.search_beam(Q, 10, 40, bw, threads=8)
    assert (found == 10).all()
    assert (np.diff(d, axis=1) >= 0).all()
    r1 = orc.recall(ix.search(Q, 10, 40, threads=8)[0], gt, 10)
    rb = orc.recall(nns, gt, 10)
    assert rb >= r1 - 0.05
    assert (nexp > 0).all()


@pytest.mark.parametrize("bw", [1, 2, 4])
def test_beam_known_answers(tmp_path, bw):
    # the hand-worked traces of tests/_helpers.py (BEAM_EXPECT)
    from _helpers import BEAM_EXPECT, write_beam_known_answer_index
    paths = write_beam_known_answer_index(str(tmp_path))
    ix = orc.Index(*paths[:2])
    q = np.zeros((1, 4), np.float32)
    nexp, ids, dists = BEAM_EXPECT[bw]
    nns, d, found, ne = ix.search_beam(q, 3, 4, bw)
    assert ne[0] == nexp and found[0] == 3
    assert nns[0].tolist() == ids and d[0].tolist() == dists
    if bw == 1:
        rn, rd, rf, re, _ = ix.search(q, 3, 4)
        assert re[0] == nexp and rn[0].tolist() == ids and rd[0].tolist() == dists
