"""Build recipe for the native parts of gustann_amd (all in-tree).

Products:
  gustann_amd/lib/libgustann_hip.so    HIP kernels (gfx950) + C ABI (include/gustann.h)
  gustann_amd/lib/libgustann_index.so  host C++ index builder / data generator
  gustann_amd/lib/search_mem           search_mem-compatible command line
  gustann_amd/lib/check_recall         check_recall-compatible command line
  oracle/liboracle_gann.so             CPU oracle (test infrastructure; built by oracle/Makefile)

Run ``python -m gustann_amd.build`` or call :func:`build_all`.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

# Contraction off: every fused multiply-add in the kernels is written out, so
# the arithmetic is exactly the one the oracle restates.  Packed FP32 is
# disabled for all HIP code.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _run(cmd, verbose):
    if verbose:
        print("+", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def build_hip(verbose=False):
    os.makedirs(LIB, exist_ok=True)
    objdir = os.path.join(ROOT, "_build")
    os.makedirs(objdir, exist_ok=True)
    from concurrent.futures import ThreadPoolExecutor
    srcs = ("gann_search_cb_u8.hip", "gann_search_cb_f32.hip", "gann_search_beam_u8.hip",
            "gann_search_beam_f32.hip", "gann_search_lut.hip", "gann_kernels.hip", "gann_knn.hip",
            "gann_build.hip", "gann_api.cpp")
    objs = [os.path.join(objdir, src.rsplit(".", 1)[0] + ".o") for src in srcs]
    with ThreadPoolExecutor(max_workers=min(len(srcs), os.cpu_count() or 4)) as ex:
        for f in [ex.submit(_run, [HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj], verbose)
                  for src, obj in zip(srcs, objs)]:
            f.result()
    out = os.path.join(LIB, "libgustann_hip.so")
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs,
          "-Wl,-soname,libgustann_hip.so"], verbose)
    os.replace(tmp, out)
    return out


def build_index(verbose=False):
    os.makedirs(LIB, exist_ok=True)
    out = os.path.join(LIB, "libgustann_index.so")
    tmp = out + ".tmp"
    _run(["g++", "-O3", "-march=x86-64-v3", "-std=c++17", "-fopenmp", "-fPIC", "-shared",
          "-Wall", "-Wextra", "-o", tmp, os.path.join(CSRC, "index_builder.cpp")], verbose)
    os.replace(tmp, out)
    return out


def build_cli(verbose=False):
    out = os.path.join(LIB, "search_mem")
    src = os.path.join(CSRC, "search_mem.cpp")
    if not os.path.exists(src):
        return None
    _run(["g++", "-O2", "-std=c++17", "-Wall", "-o", out + ".tmp", src,
          f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}", f"-L{LIB}", "-lgustann_hip",
          "-Wl,-rpath,$ORIGIN", "-pthread"], verbose)
    os.replace(out + ".tmp", out)
    return out


def build_check_recall(verbose=False):
    out = os.path.join(LIB, "check_recall")
    _run(["g++", "-O2", "-std=c++17", "-Wall", "-o", out + ".tmp", os.path.join(CSRC, "check_recall.cpp"),
          f"-I{CSRC}"], verbose)
    os.replace(out + ".tmp", out)
    return out


def build_oracle(verbose=False):
    odir = os.path.join(ROOT, "oracle")
    _run(["make", "-s", "-C", odir, "-B", "liboracle_gann.so"], verbose)
    return os.path.join(odir, "liboracle_gann.so")


def build_all(verbose=False):
    if not shutil.which(HIPCC) and not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    paths = [build_hip(verbose), build_index(verbose), build_oracle(verbose),
             build_check_recall(verbose)]
    cli = build_cli(verbose)
    if cli:
        paths.append(cli)
    return paths


if __name__ == "__main__":
    for p in build_all(verbose="-v" in sys.argv):
        print(p)
