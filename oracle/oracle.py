"""ctypes binding of the CPU oracle (liboracle_gann.so): TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, as the checker or the timed CPU baseline; the product never does.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_lib = None


class OrcIndex(C.Structure):
    _fields_ = [
        ("pages", C.c_void_p), ("num_pts", C.c_int64), ("dim", C.c_int64), ("medoid", C.c_int64),
        ("node_len", C.c_int64), ("nodes_per_page", C.c_int64), ("max_m", C.c_int64),
        ("dtype", C.c_int32),
        ("pivots", C.c_void_p), ("centroid", C.c_void_p), ("chunk_offsets", C.c_void_p),
        ("num_chunks", C.c_int32), ("codes", C.c_void_p),
        ("nav_data", C.c_void_p), ("nav_graph", C.c_void_p), ("nav_map", C.c_void_p),
        ("nav_num_node", C.c_int64), ("nav_max_m", C.c_int32), ("nav_start", C.c_int32),
    ]


def lib():
    global _lib
    if _lib is None:
        path = os.path.join(_HERE, "liboracle_gann.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run `make -C oracle`")
        L = C.CDLL(path)
        P, I32, I64 = C.c_void_p, C.c_int32, C.c_int64
        L.orc_lut_build.argtypes = [P, P, P, I32, I32, P, P]
        L.orc_query_restore.argtypes = [P, I32, P, P]
        L.orc_adc.argtypes = [P, I32, P]
        L.orc_adc.restype = C.c_float
        L.orc_adc_scan.argtypes = [P, P, P, I32, I32, P, I64, P, I32, P, I32, P, I32]
        L.orc_l2.argtypes = [P, P, I32, I32]
        L.orc_l2.restype = C.c_float
        L.orc_nav_entry_local.argtypes = [C.POINTER(OrcIndex), P, C.POINTER(I32)]
        L.orc_nav_entry_local.restype = I32
        L.orc_entry.argtypes = [C.POINTER(OrcIndex), P, C.POINTER(I32)]
        L.orc_entry.restype = I32
        L.orc_search.argtypes = [C.POINTER(OrcIndex), P, I32, P, I32, I32, P, P, P, P, I32, I32]
        L.orc_search.restype = I64
        L.orc_search_beam.argtypes = [C.POINTER(OrcIndex), P, I32, P, I32, I32, I32, P, P, P, P,
                                      I32]
        L.orc_search_beam.restype = I64
        L.orc_recall.argtypes = [P, P, I32, I32, I32]
        L.orc_recall.restype = C.c_double
        L.orc_set_pin_threads.argtypes = [I32]
        L.orc_set_pin_threads.restype = None
        _lib = L
    return _lib


def set_pin_threads(on: bool):
    """Pin worker t of every later multi-threaded call to the (t mod n)-th
    CPU the process may use (one thread per core)."""
    lib().orc_set_pin_threads(1 if on else 0)


def cpu_cores():
    """(number of CPUs this process may use, CPU model from /proc/cpuinfo)."""
    n = len(os.sched_getaffinity(0))
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return n, model


def _p(a):
    return None if a is None else a.ctypes.data


def _f32(a):
    return np.ascontiguousarray(a, np.float32)


def lut_build(pivots, centroid, chunk_offsets, q):
    """LUT [M][256] of one query (src/impl/pq.cuh:8-59)."""
    pivots, centroid, q = _f32(pivots), _f32(centroid), _f32(q)
    off = np.ascontiguousarray(chunk_offsets, np.int32)
    M = off.shape[0] - 1
    out = np.empty((M, 256), np.float32)
    lib().orc_lut_build(_p(pivots), _p(centroid), _p(off), pivots.shape[1], M, _p(q), _p(out))
    return out


def query_restore(centroid, q):
    centroid, q = _f32(centroid), _f32(q)
    out = np.empty_like(q)
    lib().orc_query_restore(_p(centroid), q.shape[0], _p(q), _p(out))
    return out


def adc(lut, code):
    lut = _f32(lut)
    code = np.ascontiguousarray(code, np.uint8)
    return float(lib().orc_adc(_p(lut), lut.shape[0], _p(code)))


def adc_scan(pivots, centroid, chunk_offsets, codes, q, ids, threads=1):
    """out[i][s] = ADC(LUT(q_i), codes[ids[i][s]]) (NaN for an id out of range)."""
    pivots, centroid, q = _f32(pivots), _f32(centroid), _f32(q)
    off = np.ascontiguousarray(chunk_offsets, np.int32)
    codes = np.ascontiguousarray(codes, np.uint8)
    ids = np.ascontiguousarray(ids, np.int32)
    nq, S = ids.shape
    out = np.empty((nq, S), np.float32)
    lib().orc_adc_scan(_p(pivots), _p(centroid), _p(off), pivots.shape[1], off.shape[0] - 1,
                       _p(codes), codes.shape[0], _p(q), nq, _p(ids), S, _p(out), threads)
    return out


def l2(q, x):
    """square_sum_32 order exact L2 (src/impl/util.cuh:26-46)."""
    q = _f32(q)
    x = np.ascontiguousarray(x)
    dt = 0 if x.dtype == np.uint8 else 1
    if dt == 1:
        x = _f32(x)
    return float(lib().orc_l2(_p(q), _p(x), dt, q.shape[0]))


def recall(res, gt, k):
    """calc_recall (bin/utils.hpp:104-116) over the first gt.shape[0] queries."""
    res = np.ascontiguousarray(res, np.int32)
    gt = np.ascontiguousarray(gt, np.int32)
    return float(lib().orc_recall(_p(res), _p(gt), gt.shape[0], gt.shape[1], k))


class Index:
    """The oracle's view of one index: pages + PQ + optional pivot graph,
    loaded from the files the reference reads."""

    def __init__(self, index_file, pq_prefix, nav_prefix="", dtype="uint8"):
        from gustann_amd.index import read_pq
        self.dtype = 0 if dtype == "uint8" else 1
        es = 1 if self.dtype == 0 else 4
        with open(index_file, "rb") as f:
            hdr = f.read(4096)
        meta = np.frombuffer(hdr[8:8 + 64], np.uint64)
        self.num_pts, self.dim, self.medoid, self.node_len, self.npp = (int(v) for v in meta[:5])
        self.max_m = (self.node_len - self.dim * es) // 4 - 1
        self.num_pages = (self.num_pts + self.npp - 1) // self.npp
        self.pages = np.fromfile(index_file, np.uint8, count=self.num_pages * 4096, offset=4096)
        pq = read_pq(pq_prefix)
        self.pivots, self.centroid = pq.pivots, pq.centroid
        self.chunk_offsets, self.codes = pq.chunk_offsets, pq.codes
        self.nav = None
        if nav_prefix:
            nd = os.path.join(nav_prefix, "nav_index.data")
            hdr = np.fromfile(nd, np.int32, count=2)
            n, d = int(hdr[0]), int(hdr[1])
            vt = np.uint8 if self.dtype == 0 else np.float32
            data = np.fromfile(nd, vt, count=n * d, offset=8).reshape(n, d)
            mapping = np.loadtxt(os.path.join(nav_prefix, "map.txt"), dtype=np.int32).reshape(-1)
            raw = np.fromfile(os.path.join(nav_prefix, "nav_index"), np.uint8)
            max_m = int(np.frombuffer(raw[8:12].tobytes(), np.uint32)[0])
            start = int(np.frombuffer(raw[12:16].tobytes(), np.uint32)[0])
            words = np.frombuffer(raw[24:].tobytes(), np.int32)
            graph = np.full((n, max_m), -1, np.int32)
            pos = 0
            for i in range(n):
                k = int(words[pos])
                graph[i, :k] = words[pos + 1:pos + 1 + k]
                pos += 1 + k
            self.nav = (np.ascontiguousarray(data), graph, mapping, max_m, start)
        self._s = self._struct()

    def _struct(self):
        s = OrcIndex()
        s.pages = _p(self.pages)
        s.num_pts, s.dim, s.medoid = self.num_pts, self.dim, self.medoid
        s.node_len, s.nodes_per_page, s.max_m = self.node_len, self.npp, self.max_m
        s.dtype = self.dtype
        s.pivots, s.centroid = _p(self.pivots), _p(self.centroid)
        s.chunk_offsets, s.num_chunks = _p(self.chunk_offsets), self.chunk_offsets.shape[0] - 1
        s.codes = _p(self.codes)
        if self.nav is not None:
            data, graph, mapping, max_m, start = self.nav
            s.nav_data, s.nav_graph, s.nav_map = _p(data), _p(graph), _p(mapping)
            s.nav_num_node, s.nav_max_m, s.nav_start = data.shape[0], max_m, start
        return s

    def nav_entry_local(self, q):
        it = C.c_int32(0)
        return int(lib().orc_nav_entry_local(C.byref(self._s), _p(_f32(q)), C.byref(it))), it.value

    def entry(self, q):
        fb = C.c_int32(0)
        return int(lib().orc_entry(C.byref(self._s), _p(_f32(q)), C.byref(fb))), fb.value

    def search(self, Q, topk, L, entries=None, threads=1, check=False):
        """Returns (nns, dists, found, n_exp, invariant_violations)."""
        Q = _f32(Q)
        nq = Q.shape[0]
        nns = np.empty((nq, topk), np.int32)
        d = np.empty((nq, topk), np.float32)
        found = np.empty(nq, np.int32)
        nexp = np.empty(nq, np.int32)
        ent = None if entries is None else np.ascontiguousarray(entries, np.int32)
        v = lib().orc_search(C.byref(self._s), _p(Q), nq, _p(ent), topk, L, _p(nns), _p(d),
                             _p(found), _p(nexp), threads, 1 if check else 0)
        return nns, d, found, nexp, int(v)

    def search_beam(self, Q, topk, L, beam_width, entries=None, threads=1):
        """Beam search with beam width >= 1 (orc_search_beam); returns
        (nns, dists, found, n_exp)."""
        Q = _f32(Q)
        nq = Q.shape[0]
        nns = np.empty((nq, topk), np.int32)
        d = np.empty((nq, topk), np.float32)
        found = np.empty(nq, np.int32)
        nexp = np.empty(nq, np.int32)
        ent = None if entries is None else np.ascontiguousarray(entries, np.int32)
        lib().orc_search_beam(C.byref(self._s), _p(Q), nq, _p(ent), topk, L, beam_width, _p(nns),
                              _p(d), _p(found), _p(nexp), threads)
        return nns, d, found, nexp
