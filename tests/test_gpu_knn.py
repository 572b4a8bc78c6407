"""Exact k-NN on the GPU (gann_knn_exact) against the CPU brute force of the
index builder (gib_brute_force): uint8 results (int8 MFMA, exact integer
distances, ties by id) must be identical, including data with massive ties
and dims that are not a multiple of 32; float results agree to rounding."""
import numpy as np
import pytest

from gustann_amd import GannError
from gustann_amd import index as gi

pytestmark = pytest.mark.gpu


def _u8(n, dim, seed, hi=256):
    r = np.random.default_rng(seed)
    return r.integers(0, hi, (n, dim), dtype=np.uint8)


@pytest.mark.parametrize("dim,k", [(128, 10), (128, 100), (100, 10), (32, 128), (256, 16)])
def test_u8_identical_to_cpu(dim, k):
    X = _u8(40000, dim, 1)
    Q = _u8(77, dim, 2).astype(np.float32)
    gi_ids, gi_d = gi.brute_force_knn_gpu(X, Q, k)
    c_ids, c_d = gi.brute_force_knn(X, Q, k, threads=8)
    assert np.array_equal(gi_ids, c_ids)
    assert np.array_equal(gi_d, c_d)


def test_u8_ties_broken_by_smaller_id():
    # 6-dim 0/1 points: only 64 distinct vectors among 20000, so ranks are
    # decided by ids almost everywhere
    X = _u8(20000, 6, 3, hi=2)
    Q = _u8(40, 6, 4, hi=2).astype(np.float32)
    g = gi.brute_force_knn_gpu(X, Q, 50)
    c = gi.brute_force_knn(X, Q, 50, threads=8)
    assert np.array_equal(g[0], c[0]) and np.array_equal(g[1], c[1])
    d = ((Q[:, None, :] - X[None, :, :].astype(np.float32)) ** 2).sum(-1)
    order = np.lexsort((np.broadcast_to(np.arange(X.shape[0]), d.shape), d), axis=1)[:, :50]
    assert np.array_equal(g[0], order)


def test_f32_matches_cpu():
    r = np.random.default_rng(5)
    X = r.standard_normal((30000, 96)).astype(np.float32)
    Q = r.standard_normal((64, 96)).astype(np.float32)
    g_ids, g_d = gi.brute_force_knn_gpu(X, Q, 10)
    c_ids, c_d = gi.brute_force_knn(X, Q, 10, threads=8)
    assert (g_ids == c_ids).mean() >= 0.999
    assert np.allclose(g_d, c_d, rtol=1e-5, atol=0)
    ref = ((Q[:, None, :].astype(np.float64) - X[None].astype(np.float64)) ** 2).sum(-1)
    assert np.allclose(g_d, np.take_along_axis(ref, g_ids, 1), rtol=1e-5)


def test_fewer_points_than_k():
    X = _u8(5, 16, 6)
    Q = _u8(3, 16, 7).astype(np.float32)
    ids, d = gi.brute_force_knn_gpu(X, Q, 10)
    assert (ids[:, 5:] == -1).all() and np.isinf(d[:, 5:]).all()
    c = gi.brute_force_knn(X, Q, 10, threads=2)
    assert np.array_equal(ids, c[0])


def test_argument_errors():
    X = _u8(100, 16, 8)
    Q = np.full((2, 16), 0.5, np.float32)
    with pytest.raises(GannError):
        gi.brute_force_knn_gpu(X, Q, 10)      # uint8 queries must be integral
    with pytest.raises(GannError):
        gi.brute_force_knn_gpu(X, np.zeros((2, 16), np.float32), 129)


@pytest.mark.parametrize("chunk", ["700", "12345"])
def test_chunks_merged_on_the_device(monkeypatch, chunk):
    # GANN_KNN_CHUNK cuts the base into chunks of that many points (43 and
    # 3 chunks here, the last one ragged): each chunk's slices are merged
    # into the running best on the device
    monkeypatch.setenv("GANN_KNN_CHUNK", chunk)
    X = _u8(30000, 64, 11)
    Q = _u8(50, 64, 12).astype(np.float32)
    for k in (10, 100):
        g = gi.brute_force_knn_gpu(X, Q, k)
        c = gi.brute_force_knn(X, Q, k, threads=8)
        assert np.array_equal(g[0], c[0]) and np.array_equal(g[1], c[1]), k
    T = _u8(20000, 6, 13, hi=2)                 # ties everywhere
    Qt = _u8(33, 6, 14, hi=2).astype(np.float32)
    g = gi.brute_force_knn_gpu(T, Qt, 40)
    c = gi.brute_force_knn(T, Qt, 40, threads=8)
    assert np.array_equal(g[0], c[0]) and np.array_equal(g[1], c[1])
    r = np.random.default_rng(15)
    F = r.standard_normal((9000, 40)).astype(np.float32)
    Qf = r.standard_normal((20, 40)).astype(np.float32)
    g_ids, g_d = gi.brute_force_knn_gpu(F, Qf, 10)
    c_ids, c_d = gi.brute_force_knn(F, Qf, 10, threads=8)
    assert (g_ids == c_ids).mean() >= 0.999
    assert np.allclose(g_d, c_d, rtol=1e-5, atol=0)
