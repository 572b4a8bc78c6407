"""The device-pointer entry point (gann_search_device_ex) on torch buffers and
stream against the CPU oracle, with entry selection on the device and with
caller-given entries (GANN_SEARCH_ENTRIES_GIVEN)."""
import numpy as np
import pytest

import oracle as orc
from gustann_amd import MODE_FUSED, MODE_FUSED_GP, MODE_STEPWISE, UINT8, GustANN, GustANNConfig
from gustann_amd import _native as N
from gustann_amd import index as gi

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def setup(tiny_u8):
    P = tiny_u8["paths"]
    g = GustANN(UINT8)
    g.init_pure_mem(GustANNConfig(P["index"], P["pq"], P["nav"]), True)
    Q = gi.read_vecs(P["query"], np.uint8).astype(np.float32)
    ix = orc.Index(P["index"], P["pq"], P["nav"])
    yield g, Q, ix
    g.close()


def _run(g, Q, k, L, mode, entries=None, beam=1):
    import torch
    dev = torch.device("cuda:0")
    nq = Q.shape[0]
    q = torch.from_numpy(np.ascontiguousarray(Q)).to(dev)
    ent = (torch.from_numpy(np.ascontiguousarray(entries, np.int32)).to(dev) if entries is not None
           else torch.full((nq,), -5, dtype=torch.int32, device=dev))
    nns = torch.full((nq, k), -5, dtype=torch.int32, device=dev)
    dd = torch.full((nq, k), -5.0, dtype=torch.float32, device=dev)
    fc = torch.full((nq,), -5, dtype=torch.int32, device=dev)
    ne = torch.full((nq,), -5, dtype=torch.int32, device=dev)
    na = torch.full((nq,), -5, dtype=torch.int32, device=dev)
    s = torch.cuda.Stream()
    m = mode | (N.SEARCH_ENTRIES_GIVEN if entries is not None else 0)
    with torch.cuda.stream(s):
        g.search_device(q.data_ptr(), nq, k, L, ent.data_ptr(), nns.data_ptr(), dd.data_ptr(), fc.data_ptr(),
                        ne.data_ptr(), na.data_ptr(), s.cuda_stream, beam_width=beam, mode=m)
    s.synchronize()
    return (nns.cpu().numpy(), dd.cpu().numpy(), fc.cpu().numpy(), ne.cpu().numpy(), na.cpu().numpy(),
            ent.cpu().numpy())


def _same(got, ref):
    nns, dd, fc, ne = got[:4]
    on, od, of, oe = ref[:4]
    assert np.array_equal(fc, of)
    assert np.array_equal(nns, on)
    assert np.array_equal(dd.view(np.uint32), od.view(np.uint32))
    assert np.array_equal(ne, oe)


@pytest.mark.parametrize("mode,L,k", [(MODE_FUSED, 64, 10), (MODE_FUSED_GP, 300, 10), (MODE_STEPWISE, 48, 10)])
def test_device_entry_point_matches_oracle(setup, mode, L, k):
    g, Q, ix = setup
    got = _run(g, Q, k, L, mode)
    assert np.array_equal(got[5], [ix.entry(q)[0] for q in Q])
    _same(got, ix.search(Q, k, L, threads=8))


@pytest.mark.parametrize("mode", [MODE_FUSED, MODE_FUSED_GP, MODE_STEPWISE])
def test_given_entries_skip_selection(setup, mode):
    g, Q, ix = setup
    rng = np.random.default_rng(5)
    ent = rng.integers(0, ix.num_pts, Q.shape[0]).astype(np.int32)
    got = _run(g, Q, 10, 80, mode, entries=ent)
    assert np.array_equal(got[5], ent)  # entries are inputs, left as given
    _same(got, ix.search(Q, 10, 80, entries=ent, threads=8))


def test_given_entry_outside_the_index_gives_an_empty_result(setup):
    g, Q, ix = setup
    ent = np.array([ix.num_pts, -1, 2**31 - 1, 0], np.int32)
    nns, dd, fc, ne, na, _ = _run(g, Q[:4], 10, 40, MODE_FUSED, entries=ent)
    assert fc[:3].tolist() == [0, 0, 0] and ne[:3].tolist() == [0, 0, 0] and na[:3].tolist() == [0, 0, 0]
    assert (nns[:3] == 0).all() and (dd[:3] == 0).all()
    _same((nns[3:], dd[3:], fc[3:], ne[3:]), [a[3:] for a in ix.search(Q[:4], 10, 40, entries=ent.clip(0, 0),
                                                                       threads=1)[:4]])
