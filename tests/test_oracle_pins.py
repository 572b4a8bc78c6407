"""Pins the CPU oracle (oracle/gann_oracle.c) against what the mathematics
fixes, independently of the oracle's own formulas: closed forms in exact or
float64 arithmetic, special cases that reduce to exact integer L2, and
known-answer cases whose expected values are worked out from the reference's
operation order (a sequential sum, a shfl_down tree, fused multiply-adds).
Each case is chosen so that a plausible slip (a dropped term, a wrong sign or
index, a transposed operand, another summation order) fails it."""
import numpy as np
import pytest
from _helpers import add_f32, fma_f32

import oracle as orc


def _closed_form_lut(piv, cen, off, q):
    piv, cen, q = (np.asarray(a, np.float64) for a in (piv, cen, q))
    M = len(off) - 1
    out = np.zeros((M, 256))
    for m in range(M):
        for i in range(off[m], off[m + 1]):
            out[m] += (q[i] - cen[i] - piv[:, i]) ** 2
    return out


def test_lut_exact_integer_special_case():
    # M = D, pivots k = 0..255 in every dim, centroid 0, integer query:
    # LUT[i][k] = (q_i - k)^2 exactly (src/impl/pq.cuh:35-43).
    rng = np.random.default_rng(1)
    D = 16
    piv = np.repeat(np.arange(256, dtype=np.float32)[:, None], D, axis=1)
    q = rng.integers(0, 256, D).astype(np.float32)
    lut = orc.lut_build(piv, np.zeros(D, np.float32), np.arange(D + 1, dtype=np.int32), q)
    expect = (q[:, None].astype(np.int64) - np.arange(256)[None, :]) ** 2
    assert np.array_equal(lut.astype(np.int64), expect)


@pytest.mark.parametrize("D,off", [(128, list(range(0, 129, 4))), (96, list(range(0, 97, 2))),
                                   (30, [0, 3, 4, 9, 9, 17, 30])])
def test_lut_matches_float64_closed_form(D, off):
    rng = np.random.default_rng(D)
    piv = rng.uniform(-16, 16, (256, D)).astype(np.float32)
    cen = rng.uniform(96, 160, D).astype(np.float32)
    for _ in range(4):
        q = rng.uniform(0, 255, D).astype(np.float32)
        got = orc.lut_build(piv, cen, np.array(off, np.int32), q).astype(np.float64)
        ref = _closed_form_lut(piv, cen, off, q)
        rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)
        assert rel.max() <= 1e-5


def test_lut_accumulates_with_fused_multiply_add():
    # Row of two dims: LUT = fma(d1, d1, fl(d0^2)).  Search for inputs where
    # the fused and the unfused forms round differently, then require the
    # fused value (the oracle's stated contraction contract).
    rng = np.random.default_rng(7)
    for _ in range(20000):
        q = rng.uniform(-4, 4, 2).astype(np.float32)
        p = rng.uniform(-4, 4, 2).astype(np.float32)
        d0, d1 = np.float32(q[0] - p[0]), np.float32(q[1] - p[1])
        fused = fma_f32(d1, d1, fma_f32(d0, d0, 0.0))
        unfused = add_f32(fma_f32(d0, d0, 0.0), np.float32(d1 * d1))
        if fused != unfused:
            break
    else:
        pytest.fail("no distinguishing input found")
    piv = np.zeros((256, 2), np.float32)
    piv[5] = p
    lut = orc.lut_build(piv, np.zeros(2, np.float32), np.array([0, 2], np.int32), q)
    assert lut[0, 5] == fused and lut[0, 5] != unfused


def test_adc_equals_exact_l2_in_special_case():
    # With the exact per-dim PQ the ADC distance of a uint8 vector is its
    # exact squared L2 distance.
    rng = np.random.default_rng(3)
    D = 32
    piv = np.repeat(np.arange(256, dtype=np.float32)[:, None], D, axis=1)
    q = rng.integers(0, 256, D).astype(np.float32)
    lut = orc.lut_build(piv, np.zeros(D, np.float32), np.arange(D + 1, dtype=np.int32), q)
    for _ in range(50):
        x = rng.integers(0, 256, D).astype(np.uint8)
        assert orc.adc(lut, x) == float(((q.astype(np.int64) - x) ** 2).sum())


def test_adc_is_sequential_from_zero():
    # LUT entries [2^24, 1, 1, 1, 1, 1, 1, 1]: summed left to right from 0,
    # every +1 is a tie at 2^24 that rounds back to even, so the result is
    # exactly 2^24 (src/impl/pure_mem.cuh:306-308); a pairwise or reversed
    # order would give 2^24 + 8 or 2^24 + 7.
    lut = np.zeros((8, 256), np.float32)
    lut[0, 1] = 2.0 ** 24
    lut[1:, 1] = 1.0
    assert orc.adc(lut, np.ones(8, np.uint8)) == 2.0 ** 24


def test_adc_scan_matches_float64():
    rng = np.random.default_rng(11)
    D, M = 64, 16
    off = np.arange(0, D + 1, 4, dtype=np.int32)
    piv = rng.uniform(-8, 8, (256, D)).astype(np.float32)
    cen = rng.uniform(0, 50, D).astype(np.float32)
    codes = rng.integers(0, 256, (1000, M), dtype=np.uint8)
    Q = rng.uniform(0, 60, (5, D)).astype(np.float32)
    ids = rng.integers(0, 1000, (5, 40), dtype=np.int32)
    ids[0, 0] = 1000  # out of range -> NaN
    got = orc.adc_scan(piv, cen, off, codes, Q, ids, threads=2)
    assert np.isnan(got[0, 0])
    for i in range(5):
        L = _closed_form_lut(piv, cen, off, Q[i])
        for s in range(40):
            if i == 0 and s == 0:
                continue
            ref = L[np.arange(M), codes[ids[i, s]]].sum()
            assert abs(got[i, s] - ref) / ref <= 1e-5


def test_l2_uint8_is_exact_integer():
    rng = np.random.default_rng(5)
    for D in (3, 32, 96, 128, 200):
        q = rng.integers(0, 256, D).astype(np.float32)
        x = rng.integers(0, 256, D).astype(np.uint8)
        assert orc.l2(q, x) == float(((q.astype(np.int64) - x) ** 2).sum())


def test_l2_follows_the_shfl_down_tree():
    # Lane partials v0 = 2^24, v8 = v16 = v24 = 1 (dims 0, 8, 16, 24 of a
    # 32-dim vector).  The tree adds v0 + v16 = 2^24 + 1 -> 2^24 (tie to
    # even), v8 + v24 = 2, then 2^24 + 2 exactly (src/impl/util.cuh:40-45).
    # A sequential sum gives 2^24, float64 gives 2^24 + 3.
    q = np.zeros(32, np.float32)
    x = np.zeros(32, np.float32)
    x[0], x[8], x[16], x[24] = 4096.0, 1.0, 1.0, 1.0
    assert orc.l2(q, x) == 2.0 ** 24 + 2


def test_l2_float_matches_float64():
    rng = np.random.default_rng(9)
    for D in (96, 128, 100):
        q = rng.normal(size=D).astype(np.float32)
        x = rng.normal(size=D).astype(np.float32)
        ref = float(((q.astype(np.float64) - x) ** 2).sum())
        assert abs(orc.l2(q, x) - ref) / ref <= 1e-5


def test_query_restore_roundtrip():
    # Integer queries survive (q - mu) + mu exactly; arbitrary floats may not,
    # and the oracle must keep both roundings rather than return q.
    rng = np.random.default_rng(2)
    cen = rng.uniform(0, 200, 64).astype(np.float32)
    qi = rng.integers(0, 256, 64).astype(np.float32)
    assert np.array_equal(orc.query_restore(cen, qi), qi)
    qf = rng.normal(size=4096).astype(np.float32) * 1e-3
    cf = np.full(4096, 1000.0, np.float32)
    expect = np.array([add_f32(np.float32(a - b), b) for a, b in zip(qf, cf)], np.float32)
    got = orc.query_restore(cf, qf)
    assert np.array_equal(got, expect) and not np.array_equal(got, qf)


def test_recall_counts_duplicates_and_zero_slots():
    # calc_recall (bin/utils.hpp:104-116): a result id in the gt set counts
    # once per occurrence; unfilled slots hold id 0.
    gt = np.array([[5, 7, 0, 9], [1, 2, 3, 4]], np.int32)
    res = np.array([[5, 5, 0], [4, 9, 9]], np.int32)
    assert orc.recall(res, gt, 3) == pytest.approx((3 + 0) / 6)
