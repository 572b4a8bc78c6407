#!/usr/bin/env python3
"""Benchmark of the GustANN MI355X search path.

Default workload (the PQ kernel microbenchmark): 10,000 f32 queries of dim
128, PQ with M = 32 subspaces x 256 centroids, 100,000,000 random 32-byte code
rows resident in HBM, 4096 uniformly random candidate ids per query.  One
step = one launch of the fused LUT-build + ADC gather-scan kernel over all
queries.  Prints one JSON line:

  value      queries/s of the kernel (inputs already resident in HBM)
  roofline   algorithmic bytes per launch / average launch time vs 8 TB/s
  cpu_baseline  the CPU oracle on a bounded sample of the same workload

``--workload search`` runs the in-memory beam search on a synthetic
uint8 mixture index instead (built on the fly; slower to set up).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "QPS @ recall@10=0.9 on 1 MI355X; ADC-scan HBM GB/s vs peak"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def adc_alg_bytes(nq, dim, S, M):
    """Algorithmic bytes of one ADC launch: per query the query vector (4*dim),
    per candidate its code row (M), its id (4) and its distance (4); once the
    static pivots, centroid and chunk map."""
    return nq * (4 * dim + S * (M + 8)) + (256 * dim * 4 + 4 * dim + 4 * dim)


def cpu_baseline_adc(pq_np, codes_host, Q, ids_host, target_s):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    threads = min(16, os.cpu_count() or 1)
    piv, cen, off = pq_np
    # calibrate on a small batch, then run about target_s of work: a prefix
    # of the queries, or whole passes over all of them when one pass is short
    n0 = min(64, Q.shape[0])
    t = time.perf_counter()
    orc.adc_scan(piv, cen, off, codes_host, Q[:n0], ids_host[:n0], threads)
    per_q = (time.perf_counter() - t) / n0
    n = int(min(Q.shape[0], max(n0, target_s / max(per_q, 1e-9))))
    # the calibration batch runs cold, so keep adding whole passes until the
    # timed work reaches target_s (a prefix shorter than all queries runs once)
    passes = 0
    t = time.perf_counter()
    while True:
        out = orc.adc_scan(piv, cen, off, codes_host, Q[:n], ids_host[:n], threads)
        passes += 1
        dt = time.perf_counter() - t
        if n < Q.shape[0] or dt >= target_s:
            break
    return {"value": passes * n / dt, "unit": "queries/s", "cores": threads, "kind": "port",
            "sample": f"{passes} pass(es) over the first {n} of the {Q.shape[0]} queries x "
                      f"{ids_host.shape[1]} ids: oracle/gann_oracle.c orc_adc_scan over the full "
                      f"host copy of the codes, {threads} threads, {dt:.1f} s"}, out


def recall_at_k(res, gt, k):
    """calc_recall (bin/utils.hpp:104-116): hits of each result slot in the set
    of the first k ground-truth ids, over the ground-truth rows."""
    hits = 0
    for r, g in zip(res, gt):
        s = set(int(x) for x in g[:k])
        hits += sum(1 for x in r[:k] if int(x) in s)
    return hits / (gt.shape[0] * k)


def traffic_from_profiles(name):
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            return json.load(f).get("traffic_bytes_per_launch")
    except Exception:
        return None


def bench_adc(args):
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
    log(f"[bench] generating {N} x {M} codes and {nq} x {S} ids on the device")
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
    value = nq / (ms / 1e3)
    alg = adc_alg_bytes(nq, dim, S, M)
    achieved = alg / (ms / 1e3) / 1e9
    log(f"[bench] {args.steps} steps: {ms:.4f} ms/step (events), wall {wall:.3f} s, "
        f"{achieved:.1f} GB/s algorithmic")

    result = {
        "metric": METRIC, "value": value, "unit": "queries/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (uniform random codes, ids and queries, seeded)",
        "config": {"workload": "pq_adc_microbench", "nq": nq, "dim": dim, "M": M, "K": 256,
                   "num_codes": N, "ids_per_query": S},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": traffic_from_profiles("adc_scan_c1_traffic.json"),
                     "alg_bytes_per_launch": alg},
    }
    if not args.no_cpu:
        log("[bench] CPU baseline (oracle) on a bounded sample")
        codes_host = codes.cpu().numpy()
        ids_host = ids.cpu().numpy()
        cpu, cpu_out = cpu_baseline_adc((piv, cen, off), codes_host, Q, ids_host, args.cpu_seconds)
        result["cpu_baseline"] = cpu
        gpu_out = out[: cpu_out.shape[0]].cpu().numpy()
        result["parity_sample_bitexact"] = bool(np.array_equal(gpu_out.view(np.uint32),
                                                               cpu_out.view(np.uint32)))
    pq.close()
    return result


def bench_search(args):
    import torch
    from gustann_amd import index as gi
    from gustann_amd.search import FLOAT, GustANN, GustANNConfig, UINT8

    u8 = args.dtype == "uint8"
    sigma = args.sigma if args.sigma > 0 else (12.0 if u8 else 0.05)
    K = args.topk
    spec = gi.DatasetSpec(name=f"mix{args.n}x{args.dim}{'' if u8 else 'f'}"
                               + (f"z{args.zipf}" if args.zipf > 0 else ""),
                          n=args.n, dim=args.dim, dtype=args.dtype, nclusters=args.nclusters,
                          sigma=sigma, R=64, L_build=100, M=args.M, nq=args.nq_search,
                          k=max(10, K), nav_n=args.nav_n, gt_nq=args.gt_nq, zipf_s=args.zipf,
                          builder=args.builder,
                          extra_queries=[{"name": a, "nq": int(b), "zipf_s": float(c), "k": int(d),
                                          "gt_nq": args.gt_nq}
                                         for a, b, c, d in (x.split(":") for x in args.extra_query_set)])
    out_dir = args.data_dir or os.path.join("/tmp", f"gann_{spec.name}_{args.nav_n}_{args.builder}")
    meta_path = os.path.join(out_dir, "meta.json")
    if os.path.exists(meta_path):
        meta = json.load(open(meta_path))
    else:
        log(f"[bench] building {spec.name} under {out_dir}")
        meta = gi.build_dataset(spec, out_dir, verbose=True)
    P = meta["paths"]
    qk = f"query_{args.query_set}" if args.query_set else "query"
    if qk not in P:
        raise SystemExit(f"query set {args.query_set!r} was not built with this index")
    Q = gi.read_vecs(P[qk], np.uint8 if u8 else np.float32).astype(np.float32)
    gt = gi.read_vecs(P[f"gt_{args.query_set}" if args.query_set else "gt"], np.int32)
    g = GustANN(UINT8 if u8 else FLOAT)
    g.init_pure_mem(GustANNConfig(P["index"], P["pq"], P["nav"]), args.placement == "hbm")
    D, M, s_el = args.dim, args.M, (1 if u8 else 4)
    dev = torch.device("cuda:0")
    rep = args.repeat
    Qr = np.tile(Q, (rep, 1))
    nq = Qr.shape[0]
    q_dev = torch.from_numpy(Qr).to(dev)
    ent = torch.empty(nq, dtype=torch.int32, device=dev)
    nns = torch.empty((nq, K), dtype=torch.int32, device=dev)
    dd = torch.empty((nq, K), dtype=torch.float32, device=dev)
    mode = {"fused": 0, "stepwise": 1, "lut": 2, "paged": 3, "gp": 4, "uring": 5}[args.mode]
    fc = torch.empty(nq, dtype=torch.int32, device=dev)
    ne = torch.empty(nq, dtype=torch.int32, device=dev)
    na = torch.empty(nq, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    rows = []
    for L in args.L:
        def step():
            g.search_device(q_dev.data_ptr(), nq, K, L, ent.data_ptr(), nns.data_ptr(), dd.data_ptr(),
                            fc.data_ptr(), ne.data_ptr(), na.data_ptr(), stream.cuda_stream,
                            beam_width=args.beam, mode=mode)
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
        res = nns[: gt.shape[0]].cpu().numpy()
        rec = recall_at_k(res, gt, K)
        rec10 = recall_at_k(res, gt, 10) if K > 10 else rec
        exps = int(ne.sum().item())
        adcs = int(na.sum().item())
        alg = exps * (D * s_el + 4) + adcs * (4 + M) + nq * (4 * D + 80)
        rows.append({"L": L, "ms": ms, "qps": nq / (ms / 1e3), "recall": rec, "recall_at_10": rec10,
                     "expansions_per_query": exps / nq, "alg_GBps": alg / (ms / 1e3) / 1e9})
        log(f"[bench] L={L} {ms:.3f} ms qps={nq / (ms / 1e3):.0f} recall@{K}={rec:.4f}")
    best = next((r for r in rows if r["recall"] >= 0.9), rows[-1])
    result = {
        "metric": METRIC, "value": best["qps"], "unit": "queries/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": best["ms"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u8/f32" if u8 else "f32",
        "data": ("synthetic uint8 Gaussian mixture" if u8 else
                 f"synthetic L2-normalised f32 Gaussian mixture (sigma {sigma})"),
        "config": {"workload": (f"in_memory_search_{args.n}x{D}_{'u8' if u8 else 'f32'}_M{M}"
                                + ("" if args.placement == "hbm" else "_host_pinned")
                                + ("" if args.mode == "fused" else f"_{args.mode}")
                                + ("" if args.beam == 1 else f"_beam{args.beam}")
                                + ("" if K == 10 else f"_top{K}")
                                + ("" if args.zipf <= 0 else f"_zipf{args.zipf}")
                                + ("" if not args.query_set else f"_queries_{args.query_set}")),
                   "nq": nq, "L": best["L"], "L_sweep": rows, "index_builder": args.builder,
                   "index_build_s": meta.get("build_s")},
        "roofline": {"bound": "hbm", "achieved": best["alg_GBps"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": best["alg_GBps"] / HBM_PEAK_GBS, "traffic": None},
    }
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as orc
        log(f"[bench] CPU baseline (oracle beam search) at L={best['L']}")
        ix = orc.Index(P["index"], P["pq"], P["nav"], dtype=args.dtype)
        threads = min(16, os.cpu_count() or 1)
        n0 = min(256, Q.shape[0])
        t = time.perf_counter()
        def cpu_search(Qs):
            if args.beam > 1:
                return ix.search_beam(Qs, K, best["L"], args.beam, threads=threads)[:3]
            return ix.search(Qs, K, best["L"], threads=threads)[:3]
        cpu_search(Q[:n0])
        per_q = (time.perf_counter() - t) / n0
        n = int(min(Q.shape[0], max(n0, args.cpu_seconds / max(per_q, 1e-9))))
        t = time.perf_counter()
        on, od, of = cpu_search(Q[:n])
        dt = time.perf_counter() - t
        result["cpu_baseline"] = {"value": n / dt, "unit": "queries/s", "cores": threads,
                                  "kind": "port",
                                  "sample": f"first {n} queries at L={best['L']}: oracle/gann_oracle.c "
                                            f"{'orc_search_beam' if args.beam > 1 else 'orc_search'}, "
                                            f"{threads} threads, {dt:.1f} s"}
        gn, gd, gf = g.search(Q[:n], n, K, best["L"], beam_width=args.beam)
        result["parity_sample_bitexact"] = bool(np.array_equal(gn, on) and np.array_equal(gf, of)
                                                and np.array_equal(gd.view(np.uint32), od.view(np.uint32)))
    g.close()
    return result


MFMA_I8_PEAK_TOPS = 5000.0  # MI355X dense int8


def bench_knn(args):
    """Exact k-NN (ground truth) of nq uint8 queries over n uint8 points
    (gann_knn_exact, int8 MFMA).  Timed end to end (base upload, kernels,
    host merge of the slices); operations counted as 2 * n * nq * dim int8
    multiply-adds."""
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
        m = max(1, min(nq, 64))
        t = time.perf_counter()
        c_ids, c_d = gi.brute_force_knn(X, Q[:m], k, threads=min(16, os.cpu_count() or 1))
        cdt = time.perf_counter() - t
        result["cpu_baseline"] = {"value": m / cdt, "unit": "queries/s",
                                  "cores": min(16, os.cpu_count() or 1), "kind": "port",
                                  "sample": f"first {m} queries: gib_brute_force, {cdt:.1f} s"}
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
    ap.add_argument("--workload", choices=["adc", "search", "copy", "knn", "gather"], default="adc")
    ap.add_argument("--knn-k", type=int, default=100)
    ap.add_argument("--copy-bytes", type=int, default=1 << 31)
    ap.add_argument("--gather-order", default="random",
                    help="gather workload: random (the ADC pattern), sorted, or band:B")
    ap.add_argument("--nq", type=int, default=10000)
    ap.add_argument("--ids-per-query", type=int, default=4096)
    ap.add_argument("--num-codes", type=int, default=100_000_000)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--n", type=int, default=1_000_000)
    ap.add_argument("--nclusters", type=int, default=1000)
    ap.add_argument("--nav-n", type=int, default=0)
    ap.add_argument("--nq-search", type=int, default=10000)
    ap.add_argument("--gt-nq", type=int, default=1000)
    ap.add_argument("--repeat", type=int, default=1)
    ap.add_argument("--L", type=int, nargs="+", default=[32, 48, 64, 96, 128])
    ap.add_argument("--data-dir", default="")
    ap.add_argument("--dtype", choices=["uint8", "float"], default="uint8")
    ap.add_argument("--dim", type=int, default=128)
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
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    if args.workload == "copy":
        res = bench_copy(args)
    else:
        res = {"adc": bench_adc, "search": bench_search, "knn": bench_knn,
               "gather": bench_gather}[args.workload](args)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
