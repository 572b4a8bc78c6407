"""GPU parity of the PQ kernels (LUT build, ADC gather-scan) against the CPU
oracle: bit-exact on identical inputs (the ADC bar of the north star is 1e-5
relative; the kernels meet it with zero difference)."""
import numpy as np
import pytest

import oracle as orc
from gustann_amd import GannError, PQSearch
from gustann_amd import index as gi

pytestmark = pytest.mark.gpu

SHAPES = [  # (dim, chunk offsets) covering every kernel specialisation
    (128, list(range(0, 129, 4))),        # M=32, 4-dim chunks: 2 words/row, unrolled LUT
    (96, list(range(0, 97, 2))),          # M=48, 2-dim chunks: 3 words/row
    (64, list(range(0, 65, 4))),          # M=16: 1 word/row
    (64, list(range(0, 65, 1))),          # M=64, 1-dim chunks: 4 words/row, generic LUT
    (30, [0, 3, 4, 9, 9, 17, 21, 25, 28, 29, 30]),  # M=10 irregular: byte path
]


def _pq(rng, D, off, n):
    piv = rng.uniform(-16, 16, (256, D)).astype(np.float32)
    cen = rng.uniform(96, 160, D).astype(np.float32)
    codes = rng.integers(0, 256, (n, len(off) - 1), dtype=np.uint8)
    return piv, cen, np.array(off, np.int32), codes


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("D,off", SHAPES)
def test_lut_build_bitexact(D, off):
    rng = np.random.default_rng(D + len(off))
    piv, cen, off, codes = _pq(rng, D, off, 100)
    pq = PQSearch.create(piv, cen, off, codes)
    Q = rng.uniform(0, 255, (17, D)).astype(np.float32)
    got = pq.lut_build(Q)
    ref = np.stack([orc.lut_build(piv, cen, off, q) for q in Q])
    assert np.array_equal(_bits(got), _bits(ref))
    pq.close()


@pytest.mark.parametrize("D,off", SHAPES)
@pytest.mark.parametrize("S", [1, 255, 1000, 4096])
def test_adc_scan_bitexact(D, off, S):
    rng = np.random.default_rng(S + D)
    n = 50_000
    piv, cen, off, codes = _pq(rng, D, off, n)
    pq = PQSearch.create(piv, cen, off, codes)
    nq = 33
    Q = rng.uniform(0, 255, (nq, D)).astype(np.float32)
    ids = rng.integers(0, n, (nq, S), dtype=np.int32)
    ids[0, 0] = 0
    ids[-1, -1] = n - 1
    got = pq.adc_scan(Q, ids)
    ref = orc.adc_scan(piv, cen, off, codes, Q, ids, threads=8)
    assert np.array_equal(_bits(got), _bits(ref))
    pq.close()


def test_adc_scan_host_rejects_out_of_range_ids():
    rng = np.random.default_rng(0)
    piv, cen, off, codes = _pq(rng, 128, list(range(0, 129, 4)), 100)
    pq = PQSearch.create(piv, cen, off, codes)
    Q = rng.uniform(0, 255, (2, 128)).astype(np.float32)
    with pytest.raises(GannError) as e:
        pq.adc_scan(Q, np.array([[0, 100], [1, 2]], np.int32))
    assert e.value.code == 1
    with pytest.raises(GannError):
        pq.adc_scan(Q, np.array([[0, -1], [1, 2]], np.int32))
    pq.close()


def test_adc_scan_device_on_torch_stream_and_nan_for_bad_ids():
    import torch
    rng = np.random.default_rng(1)
    piv, cen, off, codes = _pq(rng, 128, list(range(0, 129, 4)), 20_000)
    dev = torch.device("cuda:0")
    codes_t = torch.from_numpy(codes).to(dev)
    pq = PQSearch.create(piv, cen, off, codes_device_ptr=codes_t.data_ptr(), num_pts=codes.shape[0])
    Q = rng.uniform(0, 255, (64, 128)).astype(np.float32)
    ids = rng.integers(0, 20_000, (64, 777), dtype=np.int32)
    ids[3, 5] = 20_000
    ids[4, 6] = -7
    q_t, ids_t = torch.from_numpy(Q).to(dev), torch.from_numpy(ids).to(dev)
    out_t = torch.full((64, 777), -1.0, device=dev)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        pq.adc_scan_device(q_t.data_ptr(), 64, ids_t.data_ptr(), 777, out_t.data_ptr(), s.cuda_stream)
    s.synchronize()
    got = out_t.cpu().numpy()
    ref = orc.adc_scan(piv, cen, off, codes, Q, ids, threads=8)
    assert np.isnan(got[3, 5]) and np.isnan(got[4, 6])
    mask = ~np.isnan(ref)
    assert np.array_equal(_bits(got[mask]), _bits(ref[mask]))
    pq.close()


def test_zero_sized_calls_are_noops():
    rng = np.random.default_rng(2)
    piv, cen, off, codes = _pq(rng, 128, list(range(0, 129, 4)), 10)
    pq = PQSearch.create(piv, cen, off, codes)
    assert pq.adc_scan(np.zeros((0, 128), np.float32), np.zeros((0, 5), np.int32)).shape == (0, 5)
    assert pq.lut_build(np.zeros((0, 128), np.float32)).shape == (0, 32, 256)
    pq.close()


def test_pq_open_from_files_matches_create(tiny_u8):
    P = tiny_u8["paths"]
    t = gi.read_pq(P["pq"])
    a = PQSearch.open(P["pq"])
    b = PQSearch.create(t.pivots, t.centroid, t.chunk_offsets, t.codes)
    Q = gi.read_vecs(P["query"], np.uint8).astype(np.float32)[:20]
    ids = np.random.default_rng(3).integers(0, t.codes.shape[0], (20, 300), dtype=np.int32)
    ga, gb = a.adc_scan(Q, ids), b.adc_scan(Q, ids)
    ref = orc.adc_scan(t.pivots, t.centroid, t.chunk_offsets, t.codes, Q, ids)
    assert np.array_equal(_bits(ga), _bits(ref)) and np.array_equal(_bits(gb), _bits(ref))
    a.close()
    b.close()


def test_adc_full_size_sample():
    # The microbenchmark's full shape: 100M x 32-byte codes resident in HBM,
    # 4096 ids per query; a sample of queries is checked against the oracle
    # on the host copy of the same codes.
    import torch
    dev = torch.device("cuda:0")
    N, M, D, S = 100_000_000, 32, 128, 4096
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    codes = torch.randint(0, 256, (N, M), dtype=torch.uint8, device=dev, generator=g)
    rng = np.random.default_rng(5)
    piv = rng.uniform(-16, 16, (256, D)).astype(np.float32)
    cen = rng.uniform(96, 160, D).astype(np.float32)
    off = np.arange(0, D + 1, 4, dtype=np.int32)
    Q = rng.uniform(0, 255, (24, D)).astype(np.float32)
    ids = rng.integers(0, N, (24, S), dtype=np.int32)
    ids[0, :2] = [0, N - 1]
    pq = PQSearch.create(piv, cen, off, codes_device_ptr=codes.data_ptr(), num_pts=N)
    out = torch.empty((24, S), device=dev)
    q_t, ids_t = torch.from_numpy(Q).to(dev), torch.from_numpy(ids).to(dev)
    pq.adc_scan_device(q_t.data_ptr(), 24, ids_t.data_ptr(), S, out.data_ptr(), 0)
    torch.cuda.synchronize()
    rows = codes[torch.from_numpy(ids.ravel().astype(np.int64)).to(dev)].cpu().numpy()
    ref = orc.adc_scan(piv, cen, off, rows, Q, np.arange(24 * S, dtype=np.int32).reshape(24, S),
                       threads=8)
    assert np.array_equal(_bits(out.cpu().numpy()), _bits(ref))
    pq.close()
    del codes
    torch.cuda.empty_cache()
