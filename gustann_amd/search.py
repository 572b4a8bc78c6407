"""Host-side mirror of the reference's search interface over the C ABI.

``GustANN`` follows gustann::GustANN (src/ssd_search.hpp:29-83):
``GustANN(data_type)``, ``init_pure_mem(config, use_gpu_mem)`` and
``search(qdata, num_queries, topk, ef_search, nns, distances, found_cnt,
stats)`` with the same argument meaning; errors raise ``GannError`` where the
reference aborted, exited or threw.  ``PQSearch`` exposes the PQ tables
(src/pq_search.hpp:32-48) with the LUT build and ADC scan as kernels.
Every call runs on the GPU through libgustann_hip.so; there is no CPU path.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _native as N

UINT8 = N.UINT8
FLOAT = N.FLOAT


@dataclass
class GustANNConfig:
    """GustANNConfig (src/ssd_search.hpp:18-23)."""
    index_file: str
    pq_file_prefix: str
    nav_graph_prefix: str = ""


@dataclass
class GustANNStats:
    """GustANNStats (src/ssd_search.hpp:25-27) plus device counters."""
    run_time: float = 0.0
    entry_time: float = 0.0
    n_expansions: int = 0
    n_adc: int = 0
    alg_bytes: float = 0.0
    n_nav_fallback: int = 0


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class GustANN:
    """gustann::GustANN restricted to the PURE_MEM executor."""

    def __init__(self, data_type: int = FLOAT):
        if data_type not in (UINT8, FLOAT):
            raise ValueError("data_type must be UINT8 or FLOAT")
        self.data_type = data_type
        self._h = None
        self.info: N.IndexInfo | None = None

    def init_pure_mem(self, config: GustANNConfig, use_gpu_mem: bool = True, device_id: int = 0):
        """GustANN::init_pure_mem (src/ssd_search.cu:108-112): loads the index,
        PQ tables and optional pivot graph; use_gpu_mem selects HBM residency
        (-G) over zero-copy pinned host memory."""
        lib = N.hip_lib()
        cfg = N.Config(config.index_file.encode(), config.pq_file_prefix.encode(),
                       config.nav_graph_prefix.encode() if config.nav_graph_prefix else None,
                       self.data_type,
                       N.PLACEMENT_HBM if use_gpu_mem else N.PLACEMENT_HOST_PINNED, device_id)
        h = C.c_void_p()
        N.check(lib.gann_open(C.byref(cfg), C.byref(h)))
        self._h = h
        info = N.IndexInfo()
        N.check(lib.gann_get_info(h, C.byref(info)))
        self.info = info

    @property
    def handle(self):
        if self._h is None:
            raise N.GannError(1, "UnInited! (src/ssd_search.cu:138-139)")
        return self._h

    def search(self, qdata, num_queries: int, topk: int, ef_search: int, nns=None, distances=None,
               found_cnt=None, stats: GustANNStats | None = None, beam_width: int = 1,
               mode: int = N.MODE_FUSED, n_exp=None):
        """GustANN::search (src/ssd_search.cu:114-140).  qdata: [nq][dim] f32.
        Output arrays are filled in place when given; all are returned."""
        q = _f32(qdata).reshape(num_queries, int(self.info.dim) if self.info else -1)
        if nns is None:
            nns = np.empty((num_queries, topk), np.int32)
        if distances is None:
            distances = np.empty((num_queries, topk), np.float32)
        if found_cnt is None:
            found_cnt = np.empty(num_queries, np.int32)
        for a, dt in ((nns, np.int32), (distances, np.float32), (found_cnt, np.int32)):
            if a.dtype != dt or not a.flags.c_contiguous:
                raise ValueError("output arrays must be C-contiguous int32/float32")
        if nns.size < num_queries * topk or distances.size < num_queries * topk or found_cnt.size < num_queries:
            raise ValueError("output arrays too small")
        if n_exp is not None:
            if (not isinstance(n_exp, np.ndarray) or n_exp.dtype != np.int32
                    or not n_exp.flags.c_contiguous or n_exp.size < num_queries):
                raise ValueError("n_exp must be a C-contiguous int32 array of at least num_queries entries")
        st = N.Stats()
        ne = None if n_exp is None else n_exp.ctypes.data
        N.check(N.hip_lib().gann_search_ex(self.handle, q.ctypes.data, num_queries, topk, ef_search,
                                           beam_width, mode, nns.ctypes.data, distances.ctypes.data,
                                           found_cnt.ctypes.data, ne, C.byref(st)))
        if stats is not None:
            stats.run_time = st.run_time_s
            stats.entry_time = st.entry_time_s
            stats.n_expansions = st.n_expansions
            stats.n_adc = st.n_adc
            stats.alg_bytes = st.alg_bytes
            stats.n_nav_fallback = st.n_nav_fallback
        return nns, distances, found_cnt

    def nav_entry(self, qdata):
        """get_entry_kernel + NavGraph::translate: (base entries, pivot-local ids)."""
        q = _f32(qdata)
        nq = q.shape[0]
        ent = np.empty(nq, np.int32)
        loc = np.empty(nq, np.int32)
        N.check(N.hip_lib().gann_nav_entry(self.handle, q.ctypes.data, nq, ent.ctypes.data,
                                           loc.ctypes.data))
        return ent, loc

    def search_device(self, q_ptr, nq, topk, L, entries_ptr, nns_ptr, dists_ptr, found_ptr,
                      nexp_ptr=None, nadc_ptr=None, stream=None, beam_width=1, mode=N.MODE_FUSED):
        """Asynchronous search on device buffers (raw device pointers)."""
        N.check(N.hip_lib().gann_search_device_ex(self.handle, q_ptr, nq, topk, L, beam_width, mode,
                                                  entries_ptr, nns_ptr, dists_ptr, found_ptr,
                                                  nexp_ptr, nadc_ptr, stream))

    def search_device_noalloc(self, q_ptr, nq, topk, L, entries_ptr, nns_ptr, dists_ptr, found_ptr,
                              nexp_ptr=None, nadc_ptr=None, stream=None, beam_width=1,
                              mode=N.MODE_FUSED):
        """search_device with the kernels' scratch in the library's fixed
        device array: no device allocation (fused modes; nq * dim * 4 bytes
        at most 64 MiB - 256 B; calls that overlap on one GPU race)."""
        N.check(N.hip_lib().gann_search_device_noalloc(self.handle, q_ptr, nq, topk, L, beam_width, mode,
                                                       entries_ptr, nns_ptr, dists_ptr, found_ptr,
                                                       nexp_ptr, nadc_ptr, stream))

    def pq(self) -> "PQSearch":
        p = C.c_void_p()
        N.check(N.hip_lib().gann_handle_pq(self.handle, C.byref(p)))
        return PQSearch(p, owned=False, dim=int(self.info.dim), M=int(self.info.num_chunks))

    def close(self):
        if self._h is not None:
            N.check(N.hip_lib().gann_close(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


class PQSearch:
    """PQ tables resident on the device with the LUT build / ADC scan kernels."""

    def __init__(self, handle, owned: bool, dim: int, M: int):
        self._p = handle
        self._owned = owned
        self.dim = dim
        self.M = M

    @classmethod
    def open(cls, prefix: str, device_id: int = 0) -> "PQSearch":
        """PQSearch::read_data + init_device (src/pq_search.cu:56-185)."""
        p = C.c_void_p()
        N.check(N.hip_lib().gann_pq_open(prefix.encode(), device_id, C.byref(p)))
        from .index import read_pq_meta
        dim, M = read_pq_meta(prefix)
        return cls(p, True, dim, M)

    @classmethod
    def create(cls, pivots, centroid, chunk_offsets, codes=None, codes_device_ptr=None,
               num_pts=None, device_id: int = 0) -> "PQSearch":
        piv = _f32(pivots)
        cen = _f32(centroid)
        off = np.ascontiguousarray(chunk_offsets, np.int32)
        dim, M = piv.shape[1], off.shape[0] - 1
        p = C.c_void_p()
        if codes_device_ptr is not None:
            N.check(N.hip_lib().gann_pq_create(piv.ctypes.data, cen.ctypes.data, off.ctypes.data, dim,
                                               M, codes_device_ptr, int(num_pts), 1, device_id,
                                               C.byref(p)))
        else:
            c = np.ascontiguousarray(codes, np.uint8)
            N.check(N.hip_lib().gann_pq_create(piv.ctypes.data, cen.ctypes.data, off.ctypes.data, dim,
                                               M, c.ctypes.data, c.shape[0], 0, device_id,
                                               C.byref(p)))
        return cls(p, True, dim, M)

    def lut_build(self, q) -> np.ndarray:
        q = _f32(q).reshape(-1, self.dim)
        out = np.empty((q.shape[0], self.M, 256), np.float32)
        N.check(N.hip_lib().gann_pq_lut_build(self._p, q.ctypes.data, q.shape[0], out.ctypes.data))
        return out

    def adc_scan(self, q, ids) -> np.ndarray:
        q = _f32(q).reshape(-1, self.dim)
        ids = np.ascontiguousarray(ids, np.int32)
        if ids.ndim != 2 or ids.shape[0] != q.shape[0]:
            raise ValueError("ids must be [nq][ids_per_q]")
        out = np.empty(ids.shape, np.float32)
        N.check(N.hip_lib().gann_pq_adc_scan(self._p, q.ctypes.data, q.shape[0], ids.ctypes.data,
                                             ids.shape[1], out.ctypes.data))
        return out

    def adc_scan_device(self, q_ptr, nq, ids_ptr, ids_per_q, out_ptr, stream=None):
        N.check(N.hip_lib().gann_pq_adc_scan_device(self._p, q_ptr, nq, ids_ptr, ids_per_q, out_ptr,
                                                    stream))

    def close(self):
        if self._p is not None and self._owned:
            N.check(N.hip_lib().gann_pq_close(self._p))
        self._p = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
