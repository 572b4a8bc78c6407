"""Summarises rocprofv3 CSV output for one kernel.

  python -m gustann_amd.prof_summary --kernel pq_adc_scan_kernel \\
      --trace DIR [--fetch DIR --write DIR --copy-fetch DIR --copy-write DIR \\
      --copy-kernel copyBuffer --copy-bytes N --alg-bytes B] [--meta KEY=VALUE] [--json OUT]

--trace: a `rocprofv3 --kernel-trace --stats --output-format csv` directory
(average duration of the kernel); --fetch/--write: `--pmc FETCH_SIZE` /
`--pmc WRITE_SIZE` directories (KiB per dispatch).  With the copy-kernel
runs, each counter is scaled by copy_bytes / (what the same counter reads for
the copy), giving HBM bytes per launch.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import statistics


def _find(d, suffix):
    hits = glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True)
    if not hits:
        raise FileNotFoundError(f"no *{suffix} under {d}")
    return hits[0]


def kernel_stats(d, pattern):
    for r in csv.DictReader(open(_find(d, "kernel_stats.csv"))):
        if pattern in r["Name"]:
            return {"name": r["Name"], "calls": int(r["Calls"]), "avg_ns": float(r["AverageNs"]),
                    "min_ns": float(r["MinNs"]), "max_ns": float(r["MaxNs"])}
    raise KeyError(pattern)


def counter_per_dispatch(d, pattern, counter):
    vals = {}
    for r in csv.DictReader(open(_find(d, "counter_collection.csv"))):
        if pattern in r["Kernel_Name"] and r["Counter_Name"] == counter:
            vals[r["Dispatch_Id"]] = vals.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
    if not vals:
        raise KeyError(f"{counter} for {pattern}")
    return statistics.median(vals.values())


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--kernel", required=True)
    ap.add_argument("--trace")
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--copy-fetch")
    ap.add_argument("--copy-write")
    ap.add_argument("--copy-kernel", default="copyBuffer")
    ap.add_argument("--copy-bytes", type=float, default=float(1 << 31))
    ap.add_argument("--alg-bytes", type=float)
    ap.add_argument("--json")
    ap.add_argument("--meta", action="append", default=[],
                    help="KEY=VALUE recorded in the summary (e.g. L=2576); integer values as numbers")
    a = ap.parse_args()
    out = {"kernel": a.kernel}
    for kv in a.meta:
        k, v = kv.split("=", 1)
        out[k] = int(v) if v.lstrip("-").isdigit() else v
    if a.trace:
        out["trace"] = kernel_stats(a.trace, a.kernel)
    if a.fetch and a.write:
        fk = counter_per_dispatch(a.fetch, a.kernel, "FETCH_SIZE")
        wk = counter_per_dispatch(a.write, a.kernel, "WRITE_SIZE")
        out["FETCH_SIZE_KiB"] = fk
        out["WRITE_SIZE_KiB"] = wk
        fs = ws = 1.0
        if a.copy_fetch and a.copy_write:
            cf = counter_per_dispatch(a.copy_fetch, a.copy_kernel, "FETCH_SIZE")
            cw = counter_per_dispatch(a.copy_write, a.copy_kernel, "WRITE_SIZE")
            fs = a.copy_bytes / (cf * 1024.0)
            ws = a.copy_bytes / (cw * 1024.0)
            out["copy_FETCH_SIZE_KiB"] = cf
            out["copy_WRITE_SIZE_KiB"] = cw
        out["fetch_scale"] = fs
        out["write_scale"] = ws
        out["traffic_bytes_per_launch"] = fk * 1024.0 * fs + wk * 1024.0 * ws
        if a.alg_bytes:
            out["alg_bytes_per_launch"] = a.alg_bytes
            out["traffic_over_alg"] = out["traffic_bytes_per_launch"] / a.alg_bytes
    if a.trace and a.alg_bytes:
        out["achieved_GBps_alg"] = a.alg_bytes / (out["trace"]["avg_ns"] * 1e-9) / 1e9
    print(json.dumps(out, indent=1))
    if a.json:
        with open(a.json, "w") as f:
            json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()
