"""The fused kernels' query order (gustann_amd/csrc/gann_kernels.hip
order_bucket / query_order_kernel) restated in numpy: bucket 4095 - min(bits
>> 19, 4095) of each entry distance, a counting sort over the 4096 buckets
(exclusive scan of the counts, then each query to its bucket's next slot).
Checked against numpy's stable argsort on the float values themselves: the
result is a permutation of the queries, ordered by distance from largest to
smallest up to ties inside one bucket (distances within a factor 1 + 1/16 of
each other), so no query is taken twice or dropped and the order is
farthest-first."""
import numpy as np
import pytest


def order_bucket(d):
    b = np.asarray(d, np.float32).view(np.uint32) >> np.uint32(19)
    return (4095 - np.minimum(b, 4095)).astype(np.int64)


def query_order(d):
    bk = order_bucket(d)
    cnt = np.bincount(bk, minlength=4096)
    off = np.concatenate([[0], np.cumsum(cnt)[:-1]])
    order = np.empty(len(d), np.int64)
    for i, b in enumerate(bk):                  # slot order inside a bucket is free
        order[off[b]] = i
        off[b] += 1
    return order


@pytest.mark.parametrize("seed", range(4))
def test_order_is_a_farthest_first_permutation(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 30000))
    d = (rng.gamma(2.0, 1e5, n) * rng.choice([1.0, 0.0], n, p=[0.95, 0.05])).astype(np.float32)
    d[:3] = [0.0, np.inf, 1e30] if n >= 3 else d[:3]
    order = query_order(d)
    assert np.array_equal(np.sort(order), np.arange(n))              # a permutation
    ds = d[order].astype(np.float64)
    # non-increasing up to one bucket: a later query is never more than
    # 1 + 2^-4 farther than an earlier one
    prefix_min = np.minimum.accumulate(ds)
    assert np.all(ds <= prefix_min * (1 + 2.0 ** -4) + 1e-30)
    # and the buckets themselves are in order
    assert np.all(np.diff(order_bucket(d[order])) >= 0)


def test_bucket_is_monotone_in_the_distance():
    x = np.sort(np.random.default_rng(9).gamma(1.5, 1e4, 100000).astype(np.float32))
    assert np.all(np.diff(order_bucket(x)) <= 0)      # larger distance, earlier bucket
    assert order_bucket(np.float32(np.inf)) < order_bucket(np.float32(1.0)) < order_bucket(np.float32(0.0))
