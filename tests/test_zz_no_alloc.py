"""gann_search_device_noalloc (the allocation-free search entry point)
against gann_search_device_ex on the same device buffers: identical ids,
distances, fill counts, expansion and ADC counts, on two calls in a row
(the second smaller, so stale contents of the shared fixed scratch would
show), in every fused mode it serves; and its refusals, which the host
raises before any launch."""
import numpy as np
import pytest

from gustann_amd import (MODE_FUSED, MODE_FUSED_GP, MODE_FUSED_LUT, MODE_STEPWISE, UINT8, GannError,
                         GustANN, GustANNConfig)
from gustann_amd import index as gi

pytestmark = pytest.mark.gpu


def _device_outputs(torch, nq, k):
    dev = torch.device("cuda:0")
    return {"ent": torch.full((nq,), -7, dtype=torch.int32, device=dev),
            "nns": torch.full((nq, k), -7, dtype=torch.int32, device=dev),
            "dd": torch.full((nq, k), -7.0, dtype=torch.float32, device=dev),
            "fc": torch.full((nq,), -7, dtype=torch.int32, device=dev),
            "ne": torch.full((nq,), -7, dtype=torch.int32, device=dev),
            "na": torch.full((nq,), -7, dtype=torch.int32, device=dev)}


def _call(fn, q, nq, k, L, o, stream, beam, mode):
    fn(q.data_ptr(), nq, k, L, o["ent"].data_ptr(), o["nns"].data_ptr(), o["dd"].data_ptr(),
       o["fc"].data_ptr(), o["ne"].data_ptr(), o["na"].data_ptr(), stream.cuda_stream,
       beam_width=beam, mode=mode)


def _host(o):
    return {k: v.cpu().numpy() for k, v in o.items()}


@pytest.fixture(scope="module")
def handle(tiny_u8):
    P = tiny_u8["paths"]
    g = GustANN(UINT8)
    g.init_pure_mem(GustANNConfig(P["index"], P["pq"], P["nav"]), True)
    Q = gi.read_vecs(P["query"], np.uint8).astype(np.float32)
    yield g, Q
    g.close()


@pytest.mark.parametrize("mode,beam,L,k", [(MODE_FUSED, 1, 64, 10), (MODE_FUSED, 1, 700, 10),
                                           (MODE_FUSED_GP, 1, 200, 100), (MODE_FUSED_LUT, 1, 48, 10),
                                           (MODE_FUSED, 4, 96, 10)])
def test_noalloc_equals_device_ex_twice(handle, mode, beam, L, k):
    import torch
    g, Q = handle
    stream = torch.cuda.current_stream()
    # first call: all queries; second call: a smaller, shifted slice
    for sl in (slice(0, Q.shape[0]), slice(13, 13 + Q.shape[0] // 3)):
        Qs = np.ascontiguousarray(Q[sl])
        nq = Qs.shape[0]
        q = torch.from_numpy(Qs).cuda()
        ref = _device_outputs(torch, nq, k)
        got = _device_outputs(torch, nq, k)
        _call(g.search_device, q, nq, k, L, ref, stream, beam, mode)
        _call(g.search_device_noalloc, q, nq, k, L, got, stream, beam, mode)
        torch.cuda.synchronize()
        r, o = _host(ref), _host(got)
        assert np.array_equal(o["ent"], r["ent"])
        assert np.array_equal(o["fc"], r["fc"])
        assert np.array_equal(o["nns"], r["nns"])
        assert np.array_equal(o["dd"].view(np.uint32), r["dd"].view(np.uint32))
        assert np.array_equal(o["ne"], r["ne"]) and np.array_equal(o["na"], r["na"])
        assert (r["fc"] > 0).all()


def test_noalloc_refusals(handle):
    import torch
    g, Q = handle
    stream = torch.cuda.current_stream()
    q = torch.from_numpy(np.ascontiguousarray(Q[:4])).cuda()
    o = _device_outputs(torch, 4, 10)
    with pytest.raises(GannError, match="UNSUPPORTED"):
        _call(g.search_device_noalloc, q, 4, 10, 32, o, stream, 1, MODE_STEPWISE)
    # a query count whose q - centroid exceeds the fixed scratch is refused on
    # the host before any launch (the buffers are never touched)
    cap = ((64 << 20) - 256) // (128 * 4)
    with pytest.raises(GannError, match="INVALID.*fixed scratch"):
        _call(g.search_device_noalloc, q, cap + 1, 10, 32, o, stream, 1, MODE_FUSED)
    with pytest.raises(GannError, match="INVALID"):
        _call(g.search_device_noalloc, q, 4, 10, 32, o, stream, 0, MODE_FUSED)
