"""Builds libbrowservec_hip.so in-tree (browservec_amd/lib/) with hipcc for gfx950.

Usage: python -m browservec_amd.build  (also called by __graft_entry__.build()).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libbrowservec_hip.so")
ARCH = os.environ.get("BV_OFFLOAD_ARCH", "gfx950")

# The fused scan's instantiations are split one codec per translation unit
# (bv_scan_*.hip) so that they compile in parallel.
SCAN_CODECS = ["f32dot", "f32l2", "q8", "q4", "q1a", "q1p", "ham", "i8s", "f32dot_s", "f32l2_s"]
SOURCES = (["bv_kernels.hip"] + [f"bv_scan_{c}.hip" for c in SCAN_CODECS] +
           ["bv_ivf.hip", "bv_mq.hip", "bv_select.hip", "bv_graph.hip", "bv_api.cpp"])
HEADERS = ["bv_kernels.h", "bv_device.h", "bv_scan.h", "bv_mfma.h"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # Packed fp32 forms are disabled: plain float code must not be turned into
    # v_pk_* instructions by the backend.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
    "-I", os.path.join(ROOT, "include"),
]


# The fused scan issues each atomic from one lane and reads its result later
# (a prefetched work ticket, a slot reservation read after the re-rank's row
# loads).  The backend's atomic optimizer would rewrite every such atomic into
# a single-lane atomic plus an immediate broadcast of its result, which makes
# the wave wait for the atomic's round trip on the spot.
SCAN_FLAGS = ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"]


def _compile(src: str, obj: str) -> None:
    flags = list(COMMON)
    if src.startswith("bv_scan_"):
        flags += SCAN_FLAGS
    if src.endswith(".cpp"):
        flags = ["-x", "hip"] + flags
    cmd = [HIPCC] + flags + ["-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed for {src}")
    warn = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l and "warning:" in l)
    if warn:
        sys.stderr.write(warn + "\n")


NODE_INCLUDE = os.environ.get("BV_NODE_INCLUDE", "/usr/include/node")
NAPI_SRC = os.path.join(HERE, "napi", "bv_napi.c")
NAPI_OUT = os.path.join(LIBDIR, "browservec_napi.node")


def build_napi(verbose: bool = True) -> str | None:
    """The Node binding (N-API addon over the C ABI); skipped when the image
    has no Node headers."""
    if not os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")):
        if verbose:
            print(f"skipped {NAPI_OUT}: no node_api.h under {NODE_INCLUDE}")
        return None
    tmp = NAPI_OUT + ".tmp"
    cmd = ["gcc", "-O2", "-std=c11", "-Wall", "-Wno-unused-parameter", "-shared", "-fPIC",
           "-DNODE_GYP_MODULE_NAME=browservec_napi", "-I", NODE_INCLUDE, NAPI_SRC, "-o", tmp,
           "-L", LIBDIR, "-lbrowservec_hip", "-Wl,-rpath,$ORIGIN"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("gcc failed for the N-API addon")
    os.replace(tmp, NAPI_OUT)
    if verbose:
        print(f"built {NAPI_OUT}")
    return NAPI_OUT


def _stale(src: str, obj: str) -> bool:
    """True when obj is missing or older than its source or a shared header."""
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    deps = [os.path.join(CSRC, src)] + [os.path.join(CSRC, h) for h in HEADERS]
    deps.append(os.path.join(ROOT, "include", "browservec_hip.h"))
    return any(os.path.getmtime(d) > t for d in deps if os.path.exists(d))


BENCH_SRC = "bench_stream.hip"
BENCH_LIB = os.path.join(LIBDIR, "libbv_bench.so")


def build_bench(verbose: bool = True) -> str:
    """libbv_bench.so: the streaming-read ceiling kernel bench.py loads (not
    part of the search library)."""
    obj = os.path.join(LIBDIR, "obj", BENCH_SRC + ".o")
    _compile(BENCH_SRC, obj)
    tmp = BENCH_LIB + ".tmp"
    subprocess.run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp, obj], check=True)
    os.replace(tmp, BENCH_LIB)
    if verbose:
        print(f"built {BENCH_LIB}")
    return BENCH_LIB


def build(verbose: bool = True, incremental: bool = False) -> str:
    """Compiles every source (incremental=True: only those older than their
    inputs) and links the library and the Node addon."""
    os.makedirs(LIBDIR, exist_ok=True)
    objdir = os.path.join(LIBDIR, "obj")
    os.makedirs(objdir, exist_ok=True)
    objs = [os.path.join(objdir, s + ".o") for s in SOURCES]
    todo = [(s, o) for s, o in zip(SOURCES, objs) if not incremental or _stale(s, o)]
    workers = max(1, min(len(todo), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with cf.ThreadPoolExecutor(workers) as ex:
        list(ex.map(lambda so: _compile(*so), todo))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp] + objs
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    build_napi(verbose)
    if not incremental or _stale(BENCH_SRC, os.path.join(objdir, BENCH_SRC + ".o")):
        build_bench(verbose)
    return LIB


if __name__ == "__main__":
    build(incremental="--incremental" in sys.argv)
