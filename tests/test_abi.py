"""The C ABI library loads and exports every entry point declared in
include/gustann.h; argument errors are reported as status codes without
touching a device."""
import ctypes
import os
import re

from gustann_amd import _native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    txt = open(os.path.join(ROOT, "include", "gustann.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(gann_[a-z_]+)\s*\(", txt)))


def test_every_declared_symbol_is_exported():
    lib = N.hip_lib()
    names = declared_symbols()
    assert len(names) >= 16
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(N.ABI_SYMBOLS) == names


def test_version_and_null_argument_errors():
    lib = N.hip_lib()
    assert b"gfx950" in lib.gann_version()
    h = ctypes.c_void_p()
    assert lib.gann_open(None, ctypes.byref(h)) == 1
    assert b"index_file" in lib.gann_last_error()
    assert lib.gann_close(None) == 0
    assert lib.gann_search(None, None, 0, 10, 10, 1, None, None, None, None) == 1
    assert lib.gann_pq_adc_scan(None, None, 1, None, 1, None) == 1
    assert lib.gann_get_info(None, None) == 1


def test_index_builder_library_loads():
    lib = N.index_lib()
    for name in ("gib_vamana", "gib_pq", "gib_pq_train", "gib_brute_force", "gib_write_disk_index",
                 "gib_write_pq", "gib_write_nav", "gib_inspect", "gib_sample_ids"):
        assert hasattr(lib, name)


def test_headers_compile_for_c_and_cpp_callers(tmp_path):
    import subprocess
    inc = os.path.join(ROOT, "include")
    c_src = tmp_path / "use.c"
    c_src.write_text('#include "gustann.h"\nint main(void){gann_handle* h=0; return gann_close(h);}\n')
    cpp_src = tmp_path / "use.cpp"
    cpp_src.write_text('#include "gustann.hpp"\nint main(){gustann::GustANN a(gustann::UINT8);'
                       'gustann::GustANNConfig c; (void)c; return 0;}\n')
    for cmd in (["gcc", "-std=c11", "-Wall", "-Werror", "-fsyntax-only", f"-I{inc}", str(c_src)],
                ["g++", "-std=c++17", "-Wall", "-Werror", "-fsyntax-only", f"-I{inc}", str(cpp_src)]):
        r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        assert r.returncode == 0, r.stdout


def test_builder_and_encoder_argument_errors():
    # rejected before any device call
    import numpy as np
    lib = N.hip_lib()
    X = np.zeros((10, 8), np.uint8)
    nbr = np.zeros((10, 64), np.uint32)
    deg = np.zeros(10, np.uint32)
    med = ctypes.c_int64(0)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    args = lambda n=10, dim=8, R=16, L=20, alpha=1.2, mb=4: (p(X), n, dim, R, L, alpha, 1, mb, 0, 0, p(nbr),
                                                             p(deg), ctypes.byref(med))
    assert lib.gann_build_vamana(*args(R=65)) == 6          # UNSUPPORTED: R > 64
    assert lib.gann_build_vamana(*args(dim=257)) == 6       # UNSUPPORTED: dim > 256
    assert lib.gann_build_vamana(*args(L=0)) == 6
    assert lib.gann_build_vamana(*args(alpha=0.5)) == 1     # INVALID
    assert lib.gann_build_vamana(*args(n=0)) == 1
    assert lib.gann_build_vamana(*args(mb=0)) == 1
    assert lib.gann_build_vamana(None, 10, 8, 16, 20, 1.2, 1, 4, 0, 0, p(nbr), p(deg), ctypes.byref(med)) == 1
    assert b"NULL" in lib.gann_last_error()
    piv = np.zeros((256, 8), np.float32)
    cen = np.zeros(8, np.float32)
    codes = np.zeros((10, 2), np.uint8)
    off = np.array([0, 4, 7], np.int32)                     # does not tile [0, 8)
    assert lib.gann_pq_encode(p(X), 10, 8, 0, p(piv), p(cen), p(off), 2, 0, p(codes)) == 1
    off = np.array([0, 8], np.int32)
    X2 = np.zeros((10, 40), np.uint8)
    piv2 = np.zeros((256, 40), np.float32)
    cen2 = np.zeros(40, np.float32)
    off2 = np.array([0, 20, 40], np.int32)                  # chunks wider than 16 dims
    assert lib.gann_pq_encode(p(X2), 10, 40, 0, p(piv2), p(cen2), p(off2), 2, 0, p(codes)) == 6
    assert lib.gann_pq_encode(p(X), 10, 8, 7, p(piv), p(cen), p(off), 1, 0, p(codes)) == 1  # dtype
    cand = np.zeros(225, np.uint32)
    out = np.zeros(64, np.uint32)
    k = ctypes.c_int32(0)
    assert lib.gann_diag_robust_prune(p(X), 10, 8, 0, p(cand), 225, 1.2, 16, 0, p(out), ctypes.byref(k)) == 6
    assert lib.gann_diag_robust_prune(p(X), 10, 8, 10, p(cand), 4, 1.2, 16, 0, p(out), ctypes.byref(k)) == 1
    cand[0] = 99
    assert lib.gann_diag_robust_prune(p(X), 10, 8, 0, p(cand), 4, 1.2, 16, 0, p(out), ctypes.byref(k)) == 1
