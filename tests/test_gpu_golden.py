"""The HIP path against the committed golden fixtures (tests/golden/): every
search mode, both placements, the beam search, the entry selection and the
PQ LUT / ADC kernels must return the stored oracle outputs bit for bit."""
import numpy as np
import pytest
from test_golden import NAMES, load

from gustann_amd import (FLOAT, MODE_FUSED, MODE_FUSED_GP, MODE_FUSED_LUT, MODE_STEPWISE, MODE_STEPWISE_PAGED,
                         MODE_STEPWISE_URING, UINT8, GustANN, GustANNConfig)

pytestmark = pytest.mark.gpu

MODES = [MODE_FUSED, MODE_FUSED_LUT, MODE_FUSED_GP, MODE_STEPWISE, MODE_STEPWISE_PAGED, MODE_STEPWISE_URING]


def _open(name, pinned=False):
    spec, files, exp, Q = load(name)
    g = GustANN(UINT8 if spec["dtype"] == "uint8" else FLOAT)
    g.init_pure_mem(GustANNConfig(files["index"], files["pq"], files["nav"]), not pinned)
    return g, spec, exp, Q


def _same(got, exp, prefix, ne):
    nns, d, f = got
    assert np.array_equal(f, exp[prefix + "found"])
    assert np.array_equal(nns, exp[prefix + "nns"])
    assert np.array_equal(d.view(np.uint32), exp[prefix + "dists"].view(np.uint32))
    assert np.array_equal(ne, exp[prefix + "nexp"])


@pytest.mark.parametrize("name", NAMES)
def test_golden_entries_lut_adc(name):
    g, spec, exp, Q = _open(name)
    ent, loc = g.nav_entry(Q)
    assert np.array_equal(loc, exp["nav_local"]) and np.array_equal(ent, exp["entry"])
    pq = g.pq()
    lut = pq.lut_build(Q[:spec["nlut"]])
    assert np.array_equal(lut.view(np.uint32), exp["lut"].view(np.uint32))
    adc = pq.adc_scan(Q, exp["adc_ids"])
    assert np.array_equal(adc.view(np.uint32), exp["adc"].view(np.uint32))
    g.close()


@pytest.mark.parametrize("pinned", [False, True])
@pytest.mark.parametrize("name", NAMES)
def test_golden_search_every_mode(name, pinned):
    g, spec, exp, Q = _open(name, pinned)
    nq = Q.shape[0]
    for L, k in spec["search_cases"]:
        for mode in MODES:
            print(f"[golden] {name} pinned={pinned} L={L} k={k} mode={mode}", flush=True)
            ne = np.empty(nq, np.int32)
            got = g.search(Q, nq, k, L, n_exp=ne, mode=mode)
            _same(got, exp, f"s{L}_{k}_", ne)
    g.close()


@pytest.mark.parametrize("name", NAMES)
def test_golden_beam(name):
    g, spec, exp, Q = _open(name)
    nq = Q.shape[0]
    for w, L, k in spec["beam_cases"]:
        for mode in (MODE_FUSED, MODE_FUSED_GP):
            ne = np.empty(nq, np.int32)
            got = g.search(Q, nq, k, L, beam_width=w, n_exp=ne, mode=mode)
            _same(got, exp, f"b{w}_{L}_{k}_", ne)
    g.close()
