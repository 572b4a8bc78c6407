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
