#!/usr/bin/env python3
"""Benchmark of the GustANN MI355X in-memory search path.

Default workload, the headline "QPS @ recall@10=0.9" on one MI355X: the
100M x 128 uint8 index --
  * 100,000,000 points of a seeded Gaussian mixture (10,000 centres uniform
    in [32, 224]^128, sigma 12, rounded and clipped), 10,000 queries from the
    same mixture;
  * Vamana graph R=64, L_build=100, alpha=1.2 (the GPU builder), a
    1,000,000-node pivot graph (R=32, L=50), PQ M=32 x 256;
  * pages, codes and pivot graph resident in HBM (about 45 GB);
  * exact top-10 ground truth for all 10,000 queries;
built in this run (nothing persists between runs; a --data-dir whose
meta.json holds the same spec is reused).  The smallest L whose recall@10
over all queries reaches 0.9 is found by a coarse sweep and a step-16 scan;
then one step = one pass of the search path (entry selection on the pivot
graph + the fused beam search) over the 10,000 queries, inputs resident in
HBM, timed with HIP events on the launch stream.  One JSON line:

  value         queries/s at that L (whole job, one GPU)
  roofline      the fused search kernel alone: algorithmic bytes per launch
                (per expansion the record and the neighbours' code rows, per
                query the query and its results) / its average launch time
  cpu_baseline  the CPU oracle (the same algorithm in C) at that L on every
                core the process may use, one pinned thread per core, on a
                bounded sample of the queries
  adc_microbench  the PQ kernel microbenchmark (LUT build + ADC gather-scan
                over 100M random 32-byte code rows) with its own roofline

Other workloads: --workload search (any synthetic index), adc, knn, gather,
copy (diagnostics).
"""
from __future__ import annotations

import argparse
import dataclasses
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "QPS @ recall@10=0.9 on 1 MI355X; ADC-scan HBM GB/s vs peak"
RECALL_TARGET = 0.9
COARSE_L = (1024, 1536, 2048, 2304, 2560, 2816, 3072, 3584, 4096, 5120, 6144, 8192)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ helpers

def recall_at_k(res, gt, k):
    """calc_recall (bin/utils.hpp:104-116): hits of each result slot in the
    set of the first k ground-truth ids, over the ground-truth rows (a
    duplicated id counts once per occurrence)."""
    n = gt.shape[0]
    r = np.asarray(res[:n, :k])
    g = np.asarray(gt[:n, :k])
    return float((r[:, :, None] == g[:, None, :]).any(-1).sum()) / (n * k)


def profile_json(name):
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def cpu_info():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    return orc.cpu_cores()


def c3_spec():
    from gustann_amd import index as gi
    return gi.DatasetSpec(name="c3_100m_u8", n=100_000_000, dim=128, dtype="uint8", nclusters=10_000,
                          sigma=12.0, R=64, L_build=100, alpha=1.2, M=32, nq=10_000, k=10,
                          nav_n=1_000_000, nav_R=32, nav_L=50, gt_nq=0, builder="gpu")


def dataset(spec, data_dir=""):
    """The dataset of `spec`: reused from data_dir (or the default directory
    named by a hash of the whole spec) when its meta.json holds exactly this
    spec, else built there."""
    from gustann_amd import index as gi
    sd = dataclasses.asdict(spec)
    key = hashlib.sha1(json.dumps(sd, sort_keys=True).encode()).hexdigest()[:12]
    out_dir = data_dir or os.path.join("/tmp", f"gann_{spec.name}_{key}")
    meta_path = os.path.join(out_dir, "meta.json")
    if os.path.exists(meta_path):
        with open(meta_path) as f:
            meta = json.load(f)
        if meta.get("spec") == json.loads(json.dumps(sd)):
            log(f"[bench] reusing {out_dir}")
            return meta
        log(f"[bench] {out_dir} holds another spec: rebuilding")
    log(f"[bench] building {spec.name} under {out_dir}")
    return gi.build_dataset(spec, out_dir, verbose=True)


class DeviceSearch:
    """One open handle plus device buffers for nq queries; every launch goes
    through gann_search_device_ex on the torch stream."""

    def __init__(self, meta, Q, topk, placement="hbm"):
        import torch
        from gustann_amd.search import FLOAT, GustANN, GustANNConfig, UINT8
        P = meta["paths"]
        u8 = meta["spec"]["dtype"] == "uint8"
        self.g = GustANN(UINT8 if u8 else FLOAT)
        t = time.perf_counter()
        self.g.init_pure_mem(GustANNConfig(P["index"], P["pq"], P["nav"]), placement == "hbm")
        log(f"[bench] index open ({placement}) {time.perf_counter() - t:.1f} s")
        self.torch = torch
        dev = torch.device("cuda:0")
        self.nq, self.k = Q.shape[0], topk
        self.q = torch.from_numpy(np.ascontiguousarray(Q, np.float32)).to(dev)
        self.ent = torch.empty(self.nq, dtype=torch.int32, device=dev)
        self.nns = torch.empty((self.nq, topk), dtype=torch.int32, device=dev)
        self.dd = torch.empty((self.nq, topk), dtype=torch.float32, device=dev)
        self.fc = torch.empty(self.nq, dtype=torch.int32, device=dev)
        self.ne = torch.empty(self.nq, dtype=torch.int32, device=dev)
        self.na = torch.empty(self.nq, dtype=torch.int32, device=dev)
        self.stream = torch.cuda.current_stream(dev)
        self.dim = int(self.g.info.dim)
        self.M = int(self.g.info.num_chunks)
        self.elem = 1 if u8 else 4

    def launch(self, L, beam=1, mode=0, entries_given=False):
        from gustann_amd import _native as N
        m = mode | (N.SEARCH_ENTRIES_GIVEN if entries_given else 0)
        self.g.search_device(self.q.data_ptr(), self.nq, self.k, L, self.ent.data_ptr(), self.nns.data_ptr(),
                             self.dd.data_ptr(), self.fc.data_ptr(), self.ne.data_ptr(), self.na.data_ptr(),
                             self.stream.cuda_stream, beam_width=beam, mode=m)

    def timed(self, L, steps, warmup, **kw):
        """Average ms per launch over `steps` launches after `warmup`,
        bracketed by device synchronisations, from HIP events recorded on
        the stream the kernels run on."""
        torch = self.torch
        for _ in range(warmup):
            self.launch(L, **kw)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t = time.perf_counter()
        e0.record(self.stream)
        for _ in range(steps):
            self.launch(L, **kw)
        e1.record(self.stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps, time.perf_counter() - t

    def results(self):
        return self.nns.cpu().numpy(), self.dd.cpu().numpy(), self.fc.cpu().numpy()

    def alg_bytes(self):
        """Algorithmic bytes of the last launch: per expansion the record
        read (coordinates + degree + neighbour ids), per ADC the code row
        and the neighbour id, per query the query vector and its results."""
        exps = int(self.ne.sum().item())
        adcs = int(self.na.sum().item())
        return (exps * (self.dim * self.elem + 4) + adcs * (4 + self.M)
                + self.nq * (4 * self.dim + 8 * self.k)), exps, adcs

    def close(self):
        self.g.close()


def find_L(ds, gt, k, beam=1, mode=0, coarse=COARSE_L, step=16):
    """Smallest swept L with recall@10 >= 0.9: the coarse list until one
    reaches it, then every `step` above the last coarse L that did not.
    Returns (L or None, sweep rows)."""
    rows = []

    def rec(L):
        ds.launch(L, beam=beam, mode=mode)
        ds.torch.cuda.synchronize()
        nns = ds.nns.cpu().numpy()
        r = recall_at_k(nns, gt, 10)
        rows.append({"L": L, "recall_at_10": r})
        log(f"[bench] sweep L={L} recall@10={r:.4f}")
        return r

    prev = None
    hit = None
    for L in coarse:
        if L < k:
            continue
        if rec(L) >= RECALL_TARGET:
            hit = L
            break
        prev = L
    if hit is None:
        return None, rows
    if prev is not None:
        for L in range(prev + step, hit, step):
            if rec(L) >= RECALL_TARGET:
                return L, rows
    return hit, rows


def cpu_baseline_search(meta, Q, topk, L, beam, target_s):
    """The oracle's search (orc_search, or orc_search_beam for beam > 1) at L
    on every CPU the process may use, one pinned thread per core, over the
    first queries that take about target_s.  Returns (record, (nns, dists,
    found) of the sample)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    P = meta["paths"]
    t = time.perf_counter()
    ix = orc.Index(P["index"], P["pq"], P["nav"], dtype=meta["spec"]["dtype"])
    log(f"[bench] oracle index load {time.perf_counter() - t:.1f} s")
    cores, model = orc.cpu_cores()
    orc.set_pin_threads(True)

    def run(Qs):
        if beam > 1:
            return ix.search_beam(Qs, topk, L, beam, threads=cores)[:3]
        return ix.search(Qs, topk, L, threads=cores)[:3]

    n0 = min(Q.shape[0], 2 * cores)
    t = time.perf_counter()
    run(Q[:n0])
    per_q = (time.perf_counter() - t) / n0
    n = int(min(Q.shape[0], max(n0, target_s / max(per_q, 1e-9))))
    t = time.perf_counter()
    out = run(Q[:n])
    dt = time.perf_counter() - t
    orc.set_pin_threads(False)
    rec = {"value": n / dt, "unit": "queries/s", "cores": cores, "kind": "port",
           "sample": (f"first {n} of {Q.shape[0]} queries at L={L}, top-{topk}: oracle/gann_oracle.c "
                      f"{'orc_search_beam (beam ' + str(beam) + ')' if beam > 1 else 'orc_search'}, "
                      f"{cores} threads pinned one per core, {dt:.1f} s; CPU: {model}")}
    return rec, out


# ------------------------------------------------------------------ headline

def bench_c3(args):
    import torch
    from gustann_amd import index as gi
    spec = c3_spec()
    t0 = time.perf_counter()
    meta = dataset(spec, args.data_dir)
    build_s = time.perf_counter() - t0
    P = meta["paths"]
    Q = gi.read_vecs(P["query"], np.uint8).astype(np.float32)
    gt = gi.read_vecs(P["gt"], np.int32)
    K = 10
    ds = DeviceSearch(meta, Q, K)
    if args.L:
        L, sweep = args.L[0], []
    else:
        L, sweep = find_L(ds, gt, K)
        if L is None:
            print(json.dumps({"metric": METRIC, "value": None, "error":
                              f"recall@10 stays below {RECALL_TARGET} up to L={COARSE_L[-1]}",
                              "sweep": sweep}), flush=True)
            sys.exit(1)
    log(f"[bench] L={L}: {args.warmup} warmup + {args.steps} timed steps")
    ms, wall = ds.timed(L, args.steps, args.warmup)
    nns, dd, fc = ds.results()
    rec10 = recall_at_k(nns, gt, 10)
    # the fused search kernel alone (entries given): roofline
    ms_k, _ = ds.timed(L, args.steps, 1, entries_given=True)
    alg, exps, adcs = ds.alg_bytes()
    achieved = alg / (ms_k / 1e3) / 1e9
    value = ds.nq / (ms / 1e3)
    log(f"[bench] L={L}: {ms:.3f} ms/step ({value:.0f} QPS, recall@10 {rec10:.4f}); search kernel "
        f"{ms_k:.3f} ms, {achieved:.1f} GB/s algorithmic; {exps / ds.nq:.1f} expansions/query")
    prof = profile_json("search_cb_c3_traffic.json")
    traffic = prof.get("traffic_bytes_per_launch") if prof and prof.get("L") == L else None
    result = {
        "metric": METRIC, "value": value, "unit": "queries/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": ("synthetic: seeded uint8 Gaussian mixture (10k centres in [32,224]^128, sigma 12), "
                 "index built in this run"),
        "config": {"workload": "100M x 128 uint8 index (Vamana R=64 L=100 alpha=1.2, 1M-node pivot graph, "
                               "PQ M=32 x 256, all in HBM), 10k queries, top-10, L at recall@10 >= 0.9",
                   "num_pts": spec.n, "dim": spec.dim, "R": spec.R, "M": spec.M, "nq": ds.nq, "topk": K,
                   "L": L, "recall_at_10": rec10, "recall_queries": int(gt.shape[0]),
                   "expansions_per_query": exps / ds.nq, "L_sweep": sweep,
                   "search_kernel_ms": ms_k, "entry_selection_ms": ms - ms_k,
                   "query_order": ("queue order" if os.environ.get("GANN_QUERY_ORDER", "1").strip() == "0"
                                   else "farthest from the entry point first"),
                   "dataset_build_s": meta.get("build_s") if build_s > 60 else None,
                   "dataset_ready_s": build_s, "timed_wall_s": wall},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic, "alg_bytes_per_launch": alg,
                     "kernel": "search_cb_kernel (fused beam search; pivot table through the caches, wide lookup at L >= ~2000)"},
    }
    if not args.no_cpu:
        log(f"[bench] CPU baseline (oracle) at L={L}")
        cpu, (on, od, of) = cpu_baseline_search(meta, Q, K, L, 1, args.cpu_seconds)
        result["cpu_baseline"] = cpu
        n = on.shape[0]
        result["parity_sample_bitexact"] = bool(np.array_equal(nns[:n], on) and np.array_equal(fc[:n], of)
                                                and np.array_equal(dd[:n].view(np.uint32), od.view(np.uint32)))
    ds.close()
    del ds
    torch.cuda.empty_cache()
    if not args.no_adc:
        a = argparse.Namespace(**vars(args))
        a.cpu_seconds = args.adc_cpu_seconds
        result["adc_microbench"] = bench_adc(a, nested=True)
    return result


# ------------------------------------------------------------------ generic search

def bench_search(args):
    from gustann_amd import index as gi
    u8 = args.dtype == "uint8"
    sigma = args.sigma if args.sigma > 0 else (12.0 if u8 else 0.05)
    K = args.topk
    spec = gi.DatasetSpec(name=f"mix{args.n}x{args.dim}{'' if u8 else 'f'}"
                               + (f"z{args.zipf}" if args.zipf > 0 else ""),
                          n=args.n, dim=args.dim, dtype=args.dtype, nclusters=args.nclusters,
                          sigma=sigma, R=args.R, L_build=100, M=args.M, nq=args.nq_search,
                          k=max(10, K), nav_n=args.nav_n, gt_nq=args.gt_nq, zipf_s=args.zipf,
                          builder=args.builder,
                          extra_queries=[{"name": a, "nq": int(b), "zipf_s": float(c), "k": int(d),
                                          "gt_nq": args.gt_nq}
                                         for a, b, c, d in (x.split(":") for x in args.extra_query_set)])
    meta = dataset(spec, args.data_dir)
    P = meta["paths"]
    qk = f"query_{args.query_set}" if args.query_set else "query"
    if qk not in P:
        raise SystemExit(f"query set {args.query_set!r} was not built with this index")
    Q = gi.read_vecs(P[qk], np.uint8 if u8 else np.float32).astype(np.float32)
    gt = gi.read_vecs(P[f"gt_{args.query_set}" if args.query_set else "gt"], np.int32)
    Qr = np.tile(Q, (args.repeat, 1))
    ds = DeviceSearch(meta, Qr, K, args.placement)
    mode = {"fused": 0, "stepwise": 1, "lut": 2, "paged": 3, "gp": 4, "uring": 5}[args.mode]
    rows = []
    for L in sorted(args.L):
        ms, _ = ds.timed(L, args.steps, args.warmup, beam=args.beam, mode=mode)
        nns, _, _ = ds.results()
        alg, exps, adcs = ds.alg_bytes()
        rec = recall_at_k(nns, gt, K)
        rec10 = recall_at_k(nns, gt, 10)
        rows.append({"L": L, "ms": ms, "qps": ds.nq / (ms / 1e3), "recall": rec, "recall_at_10": rec10,
                     "expansions_per_query": exps / ds.nq, "alg_GBps": alg / (ms / 1e3) / 1e9})
        log(f"[bench] L={L} {ms:.3f} ms qps={ds.nq / (ms / 1e3):.0f} recall@{K}={rec:.4f} recall@10={rec10:.4f}")
    best = next((r for r in rows if r["recall_at_10"] >= RECALL_TARGET), None)
    result = {
        "metric": METRIC, "value": best["qps"] if best else None, "unit": "queries/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": best["ms"] if best else None,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": ("synthetic uint8 Gaussian mixture" if u8 else
                 f"synthetic L2-normalised f32 Gaussian mixture (sigma {sigma})"),
        "config": {"workload": (f"in_memory_search_{args.n}x{args.dim}_{'u8' if u8 else 'f32'}_R{args.R}_M{args.M}"
                                + ("" if args.placement == "hbm" else "_host_pinned")
                                + ("" if args.mode == "fused" else f"_{args.mode}")
                                + ("" if args.beam == 1 else f"_beam{args.beam}")
                                + ("" if K == 10 else f"_top{K}")
                                + ("" if args.zipf <= 0 else f"_zipf{args.zipf}")
                                + ("" if not args.query_set else f"_queries_{args.query_set}")),
                   "nq": ds.nq, "L": best["L"] if best else None, "L_sweep": rows,
                   "recall_queries": int(gt.shape[0]), "index_builder": args.builder,
                   "index_build_s": meta.get("build_s")},
    }
    if best:
        result["roofline"] = {"bound": "hbm", "achieved": best["alg_GBps"], "peak": HBM_PEAK_GBS,
                              "unit": "GB/s", "frac": best["alg_GBps"] / HBM_PEAK_GBS, "traffic": None}
    pick = best or rows[-1]
    if not args.no_cpu:
        ds.timed(pick["L"], 1, 0, beam=args.beam, mode=mode)
        nns, dd, fc = ds.results()
        cpu, (on, od, of) = cpu_baseline_search(meta, Q, K, pick["L"], args.beam, args.cpu_seconds)
        result["cpu_baseline"] = cpu
        n = on.shape[0]
        result["parity_sample_bitexact"] = bool(np.array_equal(nns[:n], on) and np.array_equal(fc[:n], of)
                                                and np.array_equal(dd[:n].view(np.uint32), od.view(np.uint32)))
    ds.close()
    return result


# ------------------------------------------------------------------ PQ microbenchmark

def adc_alg_bytes(nq, dim, S, M):
    """Algorithmic bytes of one ADC launch: per query the query vector (4*dim),
    per candidate its code row (M), its id (4) and its distance (4); once the
    static pivots, centroid and chunk map."""
    return nq * (4 * dim + S * (M + 8)) + (256 * dim * 4 + 4 * dim + 4 * dim)


def cpu_baseline_adc(pq_np, codes_host, Q, ids_host, target_s):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    cores, model = orc.cpu_cores()
    orc.set_pin_threads(True)
    piv, cen, off = pq_np
    n0 = min(64, Q.shape[0])
    t = time.perf_counter()
    orc.adc_scan(piv, cen, off, codes_host, Q[:n0], ids_host[:n0], cores)
    per_q = (time.perf_counter() - t) / n0
    n = int(min(Q.shape[0], max(n0, target_s / max(per_q, 1e-9))))
    passes = 0
    t = time.perf_counter()
    while True:
        out = orc.adc_scan(piv, cen, off, codes_host, Q[:n], ids_host[:n], cores)
        passes += 1
        dt = time.perf_counter() - t
        if n < Q.shape[0] or dt >= target_s:
            break
    orc.set_pin_threads(False)
    return {"value": passes * n / dt, "unit": "queries/s", "cores": cores, "kind": "port",
            "sample": f"{passes} pass(es) over the first {n} of the {Q.shape[0]} queries x "
                      f"{ids_host.shape[1]} ids: oracle/gann_oracle.c orc_adc_scan over the full "
                      f"host copy of the codes, {cores} threads pinned one per core, {dt:.1f} s; "
                      f"CPU: {model}"}, out


def bench_adc(args, nested=False):
    """PQ kernel microbenchmark: 10k f32 queries of dim 128, PQ M=32 x 256,
    100M uniformly random 32-byte code rows in HBM, 4096 random ids per
    query; one step = one launch of the LUT-build + ADC gather-scan kernel."""
    import torch
    from gustann_amd.search import PQSearch

    nq, dim, M, S, N = args.nq, 128, 32, args.ids_per_query, args.num_codes
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(2024)
    Q = rng.uniform(0, 255, size=(nq, dim)).astype(np.float32)
    piv = rng.uniform(-16, 16, size=(256, dim)).astype(np.float32)
    cen = rng.uniform(96, 160, size=dim).astype(np.float32)
    off = np.arange(0, dim + 1, dim // M, dtype=np.int32)
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    log(f"[bench] ADC microbenchmark: {N} x {M} codes and {nq} x {S} ids generated on the device")
    codes = torch.randint(0, 256, (N, M), dtype=torch.uint8, device=dev, generator=g)
    ids = torch.randint(0, N, (nq, S), dtype=torch.int32, device=dev, generator=g)
    q_dev = torch.from_numpy(Q).to(dev)
    out = torch.empty((nq, S), dtype=torch.float32, device=dev)
    pq = PQSearch.create(piv, cen, off, codes_device_ptr=codes.data_ptr(), num_pts=N)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream

    def step():
        pq.adc_scan_device(q_dev.data_ptr(), nq, ids.data_ptr(), S, out.data_ptr(), sp)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    alg = adc_alg_bytes(nq, dim, S, M)
    achieved = alg / (ms / 1e3) / 1e9
    log(f"[bench] ADC: {args.steps} steps, {ms:.4f} ms/step, {achieved:.1f} GB/s algorithmic")
    prof = profile_json("adc_scan_c1_traffic.json")
    result = {
        "metric": "PQ LUT build + ADC gather-scan: queries/s (4096 candidates each)", "value": nq / (ms / 1e3),
        "unit": "queries/s", "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
        "dtype": "f32", "data": "synthetic (uniform random codes, ids and queries, seeded)",
        "config": {"workload": "pq_adc_microbench", "nq": nq, "dim": dim, "M": M, "K": 256,
                   "num_codes": N, "ids_per_query": S, "timed_wall_s": wall},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": prof.get("traffic_bytes_per_launch") if prof else None,
                     "alg_bytes_per_launch": alg, "kernel": "pq_adc_scan_kernel"},
    }
    if not nested:
        result.update({"metric": METRIC, "n_gpus": 1, "higher_is_better": True, "scaling": "weak",
                       "vs_baseline": None})
    if not args.no_cpu and args.cpu_seconds > 0:
        log("[bench] ADC CPU baseline (oracle) on a bounded sample")
        codes_host = codes.cpu().numpy()
        ids_host = ids.cpu().numpy()
        cpu, cpu_out = cpu_baseline_adc((piv, cen, off), codes_host, Q, ids_host, args.cpu_seconds)
        result["cpu_baseline"] = cpu
        gpu_out = out[: cpu_out.shape[0]].cpu().numpy()
        result["parity_sample_bitexact"] = bool(np.array_equal(gpu_out.view(np.uint32),
                                                               cpu_out.view(np.uint32)))
    pq.close()
    del codes, ids, out
    torch.cuda.empty_cache()
    return result


# ------------------------------------------------------------------ diagnostics

MFMA_I8_PEAK_TOPS = 5000.0  # MI355X dense int8


def bench_knn(args):
    """Exact k-NN (ground truth) of nq uint8 queries over n uint8 points
    (gann_knn_exact, int8 MFMA).  Timed end to end (base upload, kernels,
    the merge of the slices on the device, result download); operations
    counted as 2 * n * nq * dim int8 multiply-adds."""
    import torch  # noqa: F401  (device runtime first)
    from gustann_amd import index as gi
    n, dim, nq, k = args.n, args.dim, args.nq, args.knn_k
    r = np.random.default_rng(7)
    X = r.integers(0, 256, (n, dim), dtype=np.uint8)
    Q = r.integers(0, 256, (nq, dim), dtype=np.uint8).astype(np.float32)
    for _ in range(args.warmup):
        gi.brute_force_knn_gpu(X, Q, k)
    t = time.perf_counter()
    for _ in range(args.steps):
        ids, d = gi.brute_force_knn_gpu(X, Q, k)
    dt = (time.perf_counter() - t) / args.steps
    ops = 2.0 * n * nq * dim
    result = {
        "metric": "exact k-NN queries/s (ground truth)", "value": nq / dt, "unit": "queries/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": dt * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "i8",
        "data": "synthetic uniform uint8",
        "config": {"workload": f"exact_knn_{n}x{dim}_u8_nq{nq}_k{k}"},
        "roofline": {"bound": "mfma", "achieved": ops / dt / 1e12, "peak": MFMA_I8_PEAK_TOPS,
                     "unit": "TOP/s", "frac": ops / dt / 1e12 / MFMA_I8_PEAK_TOPS, "traffic": None},
    }
    if not args.no_cpu:
        cores, model = cpu_info()
        m = max(1, min(nq, 64))
        t = time.perf_counter()
        c_ids, c_d = gi.brute_force_knn(X, Q[:m], k, threads=cores)
        cdt = time.perf_counter() - t
        result["cpu_baseline"] = {"value": m / cdt, "unit": "queries/s", "cores": cores, "kind": "port",
                                  "sample": f"first {m} queries: gib_brute_force, {cdt:.1f} s; CPU: {model}"}
        result["parity_sample_bitexact"] = bool(np.array_equal(c_ids, ids[:m]) and
                                                np.array_equal(c_d, d[:m]))
    return result


def bench_gather(args):
    """The ADC microbenchmark's memory access alone (gann_diag_gather_rows):
    the same 100M x 32-byte codes and 10k x 4096 ids (same seeds as the adc
    workload), every row read and folded, no LUT and no arithmetic.  Its time
    is the ceiling of the ADC scan on this access pattern.

    --gather-order reorders the same requests before timing: "band:B" groups
    all requests by id >> B (band-major, the order inside a band kept), i.e.
    every query's rows of one 2^B-row band of the table are read before the
    next band's; "sorted" sorts all requests by id.  They measure how much of
    the random-order time is line re-fetches that an order sharing lines
    across queries would save."""
    import ctypes as C
    import torch
    from gustann_amd import _native as N

    nq, M, S, N_ = args.nq, 32, args.ids_per_query, args.num_codes
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    codes = torch.randint(0, 256, (N_, M), dtype=torch.uint8, device=dev, generator=g)
    ids = torch.randint(0, N_, (nq, S), dtype=torch.int32, device=dev, generator=g)
    order = args.gather_order
    if order == "sorted":
        ids = torch.sort(ids.view(-1)).values.view(nq, S).contiguous()
    elif order.startswith("band:"):
        shift = int(order.split(":", 1)[1])
        if not 0 <= shift < 31:
            raise SystemExit("--gather-order band:B needs 0 <= B < 31")
        perm = torch.argsort((ids.view(-1) >> shift).to(torch.int64), stable=True)
        ids = ids.view(-1)[perm].view(nq, S).contiguous()
        del perm
    elif order != "random":
        raise SystemExit("--gather-order is random, sorted or band:B")
    out = torch.empty((nq, S), dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    lib = N.hip_lib()

    def step():
        N.check(lib.gann_diag_gather_rows(C.c_void_p(codes.data_ptr()), N_, M, C.c_void_p(ids.data_ptr()),
                                          nq * S, C.c_void_p(out.data_ptr()), C.c_void_p(stream.cuda_stream)))

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    rows = nq * S
    return {"workload": "gather_rows_adc_pattern", "order": order, "rows": rows, "row_bytes": M,
            "ms_per_launch": ms, "rows_per_s": rows / (ms / 1e3),
            "row_bytes_GBps": rows * M / (ms / 1e3) / 1e9,
            "line_bytes_GBps": rows * 128 / (ms / 1e3) / 1e9}


def bench_copy(args):
    """Calibration kernel for the HBM traffic counters: one device-to-device
    copy of a buffer of known size (reads and writes copy_bytes each)."""
    import torch
    n = args.copy_bytes
    dev = torch.device("cuda:0")
    src = torch.ones(n, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    return {"workload": "copy", "copy_bytes": n, "ms_per_copy": ms,
            "GBps_read_plus_write": 2 * n / (ms / 1e3) / 1e9}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=["c3", "adc", "search", "copy", "knn", "gather"], default="c3")
    ap.add_argument("--knn-k", type=int, default=100)
    ap.add_argument("--copy-bytes", type=int, default=1 << 31)
    ap.add_argument("--gather-order", default="random",
                    help="gather workload: random (the ADC pattern), sorted, or band:B")
    ap.add_argument("--nq", type=int, default=10000)
    ap.add_argument("--ids-per-query", type=int, default=4096)
    ap.add_argument("--num-codes", type=int, default=100_000_000)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--adc-cpu-seconds", type=float, default=4.0,
                    help="CPU sample of the ADC microbenchmark nested in the c3 line")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-adc", action="store_true", help="c3: leave out the nested ADC microbenchmark")
    ap.add_argument("--n", type=int, default=1_000_000)
    ap.add_argument("--nclusters", type=int, default=1000)
    ap.add_argument("--nav-n", type=int, default=0)
    ap.add_argument("--nq-search", type=int, default=10000)
    ap.add_argument("--gt-nq", type=int, default=0, help="ground truth for the first N queries (0 = all)")
    ap.add_argument("--repeat", type=int, default=1)
    ap.add_argument("--L", type=int, nargs="+", default=[],
                    help="search: the L values to time; c3: a fixed L instead of the sweep")
    ap.add_argument("--data-dir", default="")
    ap.add_argument("--dtype", choices=["uint8", "float"], default="uint8")
    ap.add_argument("--dim", type=int, default=128)
    ap.add_argument("--R", type=int, default=64)
    ap.add_argument("--M", type=int, default=32)
    ap.add_argument("--sigma", type=float, default=0.0, help="0 = 12 (uint8) / 0.05 (float)")
    ap.add_argument("--placement", choices=["hbm", "pinned"], default="hbm")
    ap.add_argument("--mode", choices=["fused", "stepwise", "lut", "paged", "gp", "uring"], default="fused")
    ap.add_argument("--beam", type=int, default=1)
    ap.add_argument("--topk", type=int, default=10)
    ap.add_argument("--zipf", type=float, default=0.0, help="> 0: query clusters ~ Zipf(s)")
    ap.add_argument("--builder", choices=["cpu", "gpu"], default="cpu",
                    help="index construction: host Vamana, or the GPU builder (uint8)")
    ap.add_argument("--extra-query-set", action="append", default=[],
                    help="NAME:NQ:ZIPF_S:K -- another query set (and top-K ground truth) built with the index")
    ap.add_argument("--query-set", default="", help="search with the extra query set NAME")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU (queries shard across "
                                   "GPUs with no collective, so one GPU's figure is the unit); "
                                   "--gpus must be 1"}))
        sys.exit(2)
    if args.workload == "search" and not args.L:
        args.L = [32, 48, 64, 96, 128]
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    if args.workload == "copy":
        res = bench_copy(args)
    else:
        res = {"c3": bench_c3, "adc": bench_adc, "search": bench_search, "knn": bench_knn,
               "gather": bench_gather}[args.workload](args)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
