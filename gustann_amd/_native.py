"""ctypes bindings of libgustann_hip.so (include/gustann.h) and
libgustann_index.so.  Loading fails loudly when a library is missing: there
is no pure-Python fallback for any search path."""
from __future__ import annotations

import ctypes as C
import os

_LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")

GANN_OK = 0
ERR_NAMES = {1: "INVALID", 2: "IO", 3: "FORMAT", 4: "HIP", 5: "NOMEM", 6: "UNSUPPORTED"}

UINT8, FLOAT = 0, 1
PLACEMENT_HBM, PLACEMENT_HOST_PINNED = 0, 1
MODE_FUSED, MODE_STEPWISE, MODE_FUSED_LUT, MODE_STEPWISE_PAGED, MODE_FUSED_GP, MODE_STEPWISE_URING = 0, 1, 2, 3, 4, 5
SEARCH_ENTRIES_GIVEN = 0x100  # OR'ed into a device-entry mode: entries are inputs

# Every symbol declared in include/gustann.h.
ABI_SYMBOLS = (
    "gann_last_error", "gann_version", "gann_open", "gann_close", "gann_get_info",
    "gann_search", "gann_search_ex", "gann_search_device", "gann_search_device_ex",
    "gann_search_device_noalloc", "gann_nav_entry",
    "gann_pq_open", "gann_pq_create", "gann_pq_close", "gann_handle_pq",
    "gann_pq_lut_build", "gann_pq_adc_scan", "gann_pq_adc_scan_device", "gann_knn_exact",
    "gann_diag_gather_rows", "gann_build_vamana", "gann_diag_robust_prune", "gann_pq_encode",
)


class GannError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{ERR_NAMES.get(code, code)}] {msg}")
        self.code = code


class Config(C.Structure):
    _fields_ = [("index_file", C.c_char_p), ("pq_prefix", C.c_char_p), ("nav_prefix", C.c_char_p),
                ("dtype", C.c_int32), ("placement", C.c_int32), ("device_id", C.c_int32)]


class Stats(C.Structure):
    _fields_ = [("run_time_s", C.c_double), ("entry_time_s", C.c_double),
                ("n_expansions", C.c_int64), ("n_adc", C.c_int64), ("alg_bytes", C.c_double),
                ("n_nav_fallback", C.c_int64)]


class IndexInfo(C.Structure):
    _fields_ = [("num_pts", C.c_int64), ("dim", C.c_int64), ("medoid", C.c_int64),
                ("max_m", C.c_int64), ("node_len", C.c_int64), ("nodes_per_page", C.c_int64),
                ("num_pages", C.c_int64), ("dtype", C.c_int32), ("num_chunks", C.c_int32),
                ("nav_num_node", C.c_int64), ("nav_max_m", C.c_int32), ("nav_start", C.c_int32)]


_P = C.c_void_p
_I32 = C.c_int32
_I64 = C.c_int64

_SIGS = {
    "gann_last_error": (C.c_char_p, []),
    "gann_version": (C.c_char_p, []),
    "gann_open": (C.c_int, [C.POINTER(Config), C.POINTER(_P)]),
    "gann_close": (C.c_int, [_P]),
    "gann_get_info": (C.c_int, [_P, C.POINTER(IndexInfo)]),
    "gann_search": (C.c_int, [_P, _P, _I32, _I32, _I32, _I32, _P, _P, _P, C.POINTER(Stats)]),
    "gann_search_ex": (C.c_int, [_P, _P, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P,
                                 C.POINTER(Stats)]),
    "gann_search_device": (C.c_int, [_P, _P, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P]),
    "gann_diag_gather_rows": (C.c_int, [_P, _I64, _I32, _P, _I64, _P, _P]),
    "gann_knn_exact": (C.c_int, [_P, _I64, _I32, _I32, _P, _I32, _I32, _I32, _P, _P]),
    "gann_build_vamana": (C.c_int, [_P, _I64, _I32, _I32, _I32, C.c_float, C.c_uint64, _I64, _I32,
                                    _I32, _P, _P, C.POINTER(_I64)]),
    "gann_pq_encode": (C.c_int, [_P, _I64, _I32, _I32, _P, _P, _P, _I32, _I32, _P]),
    "gann_diag_robust_prune": (C.c_int, [_P, _I64, _I32, _I64, _P, _I32, C.c_float, _I32, _I32, _P,
                                         C.POINTER(_I32)]),
    "gann_search_device_ex": (C.c_int, [_P, _P, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P,
                                        _P, _P]),
    "gann_search_device_noalloc": (C.c_int, [_P, _P, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P,
                                             _P, _P, _P]),
    "gann_nav_entry": (C.c_int, [_P, _P, _I32, _P, _P]),
    "gann_pq_open": (C.c_int, [C.c_char_p, _I32, C.POINTER(_P)]),
    "gann_pq_create": (C.c_int, [_P, _P, _P, _I32, _I32, _P, _I64, _I32, _I32, C.POINTER(_P)]),
    "gann_pq_close": (C.c_int, [_P]),
    "gann_handle_pq": (C.c_int, [_P, C.POINTER(_P)]),
    "gann_pq_lut_build": (C.c_int, [_P, _P, _I32, _P]),
    "gann_pq_adc_scan": (C.c_int, [_P, _P, _I32, _P, _I32, _P]),
    "gann_pq_adc_scan_device": (C.c_int, [_P, _P, _I32, _P, _I32, _P, _P]),
}

_hip = None
_index = None


def lib_path(name: str) -> str:
    return os.path.join(_LIB_DIR, name)


def _preload_torch_hip_runtime():
    """PyTorch-ROCm wheels ship their own libamdhip64 with the same SONAME
    (libamdhip64.so.7) as /opt/rocm's.  Loading ours first would bring a second
    HIP runtime into the process once torch is imported, and the second one
    finds no device.  When torch is installed, load its runtime first so that
    libgustann_hip.so binds to it by SONAME and the process has one runtime."""
    import importlib.util
    spec = importlib.util.find_spec("torch")
    if spec is None or not spec.submodule_search_locations:
        return
    for loc in spec.submodule_search_locations:
        cand = os.path.join(loc, "lib", "libamdhip64.so")
        if os.path.exists(cand):
            C.CDLL(cand, mode=C.RTLD_GLOBAL)
            return


def hip_lib():
    """libgustann_hip.so, loaded once.  Raises if it has not been built."""
    global _hip
    if _hip is None:
        path = lib_path("libgustann_hip.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run `python -m gustann_amd.build` first "
                               "(the search path has no CPU fallback)")
        _preload_torch_hip_runtime()
        lib = C.CDLL(path)
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _hip = lib
    return _hip


def check(rc: int):
    if rc != GANN_OK:
        raise GannError(rc, hip_lib().gann_last_error().decode(errors="replace"))


_IDX_SIGS = {
    "gib_last_error": (C.c_char_p, []),
    "gib_set_verbose": (None, [C.c_int]),
    "gib_gen_mixture_u8": (C.c_int, [_I64, _I64, _I64, C.c_uint64, C.c_uint64, C.c_double,
                                     C.c_double, C.c_double, _P, _P, _P, C.c_int]),
    "gib_gen_mixture_f32": (C.c_int, [_I64, _I64, _I64, C.c_uint64, C.c_uint64, C.c_double, _P,
                                      _P, _P, C.c_int]),
    "gib_zipf_clusters": (C.c_int, [_I64, _I64, C.c_double, C.c_uint64, _P]),
    "gib_vamana": (C.c_int, [_P, _I64, _I64, C.c_int, _I64, _I64, C.c_float, C.c_uint64, C.c_int,
                             _P, _P, C.POINTER(_I64)]),
    "gib_pq": (C.c_int, [_P, _I64, _I64, C.c_int, C.c_int, _I64, C.c_int, C.c_uint64, C.c_int,
                         _P, _P, _P, _P]),
    "gib_pq_train": (C.c_int, [_P, _I64, _I64, C.c_int, C.c_int, _I64, C.c_int, C.c_uint64, C.c_int,
                               _P, _P, _P]),
    "gib_sample_ids": (C.c_int, [_I64, _I64, _P]),
    "gib_brute_force": (C.c_int, [_P, _I64, _P, _I64, _I64, C.c_int, _I64, _P, _P, C.c_int]),
    "gib_write_disk_index": (C.c_int, [C.c_char_p, _P, _I64, _I64, _I64, _I64, _I64, _P, _P]),
    "gib_write_pq": (C.c_int, [C.c_char_p, _P, _P, _P, _I32, _I32, _P, _I64]),
    "gib_write_nav": (C.c_int, [C.c_char_p, _P, _I64, _I64, _I64, _P, _P, _I64, _I32, _P]),
    "gib_write_vecs": (C.c_int, [C.c_char_p, _I64, _I64, _I64, _P]),
    "gib_inspect": (C.c_int, [C.c_char_p, C.c_char_p, C.c_char_p, _I64, _P]),
}


def index_lib():
    """libgustann_index.so (host index builder), loaded once."""
    global _index
    if _index is None:
        path = lib_path("libgustann_index.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run `python -m gustann_amd.build` first")
        lib = C.CDLL(path)
        for name, (res, args) in _IDX_SIGS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _index = lib
    return _index


def icheck(rc: int):
    if rc != 0:
        raise RuntimeError(index_lib().gib_last_error().decode(errors="replace"))
