"""The diagnostic row gather (gann_diag_gather_rows): each output is the XOR
of the 32-bit words of the id's row; ids outside the table read row 0."""
import ctypes as C

import numpy as np
import pytest

from gustann_amd import GannError
from gustann_amd import _native as N

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("row_bytes", [16, 32, 48, 64])
def test_gather_folds_rows(row_bytes):
    import torch
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(row_bytes)
    rows = rng.integers(0, 256, (5000, row_bytes), dtype=np.uint8)
    ids = rng.integers(-3, 5003, 20011).astype(np.int32)
    r_t = torch.from_numpy(rows).to(dev)
    i_t = torch.from_numpy(ids).to(dev)
    o_t = torch.empty(ids.size, dtype=torch.int32, device=dev)
    N.check(N.hip_lib().gann_diag_gather_rows(C.c_void_p(r_t.data_ptr()), rows.shape[0], row_bytes,
                                              C.c_void_p(i_t.data_ptr()), ids.size,
                                              C.c_void_p(o_t.data_ptr()), None))
    torch.cuda.synchronize()
    safe = np.where((ids >= 0) & (ids < rows.shape[0]), ids, 0)
    want = np.bitwise_xor.reduce(rows.view(np.uint32)[safe], axis=1)
    assert np.array_equal(o_t.cpu().numpy().view(np.uint32), want)


def test_gather_rejects_row_size():
    with pytest.raises(GannError):
        N.check(N.hip_lib().gann_diag_gather_rows(None, 10, 24, None, 1, None, None))
