import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def _ensure_built():
    libs = [os.path.join(ROOT, "gustann_amd", "lib", "libgustann_hip.so"),
            os.path.join(ROOT, "gustann_amd", "lib", "libgustann_index.so"),
            os.path.join(ROOT, "oracle", "liboracle_gann.so")]
    if not all(os.path.exists(p) for p in libs):
        from gustann_amd import build
        build.build_all()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")
    _ensure_built()


@pytest.fixture(scope="session")
def tiny_u8(tmp_path_factory):
    """20k x 128 uint8 mixture, Vamana R=32, PQ M=32 (4-dim chunks), 2k-node pivot graph."""
    from gustann_amd import index as gi
    spec = gi.DatasetSpec(name="tiny_u8", n=20000, dim=128, nclusters=100, R=32, L_build=64, M=32,
                          nq=200, k=10, nav_n=2000, pq_sample=20000, pq_iters=8)
    return gi.build_dataset(spec, str(tmp_path_factory.mktemp("tiny_u8")))


@pytest.fixture(scope="session")
def tiny_f32(tmp_path_factory):
    """8k x 96 float (L2-normalised) mixture, Vamana R=64, PQ M=48 (2-dim chunks), pivot graph."""
    from gustann_amd import index as gi
    spec = gi.DatasetSpec(name="tiny_f32", n=8000, dim=96, dtype="float", nclusters=64, sigma=0.3,
                          R=64, L_build=64, M=48, nq=150, k=10, nav_n=800, pq_sample=8000,
                          pq_iters=6)
    return gi.build_dataset(spec, str(tmp_path_factory.mktemp("tiny_f32")))
