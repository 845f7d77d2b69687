"""Builds libbusfill.so (all HIP sources, gfx950 only) in-tree.

Usage: python bus-fill_amd/build.py [--verbose]
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libbusfill.so")
BENCH_LIB = os.path.join(LIBDIR, "libbusfill_bench.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["bf_api.hip", "bf_gemm_mfma.hip", "bf_gemm_dot2.hip", "bf_gemm_lds.hip", "bf_gemm_slab.hip", "bf_gemm_split.hip", "bf_gemm_dense.hip", "bf_simple.hip", "bf_gemm_q8.hip", "bf_ggml.hip",
           "bf_gguf.cpp"]

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 anywhere in the device code.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Wall", "-Wextra", "-Werror", "-Wno-unused-parameter",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # the first kernel arguments arrive in SGPRs at wave launch instead of through
    # a load from the kernarg segment (saves one memory round trip per launch)
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning is expected.
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{err}")
    if verbose and err:
        print(err, file=sys.stderr)


def _jobs():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    cap = os.environ.get("MAX_JOBS")
    return max(1, min(n, int(cap) if cap and cap.isdigit() else 16))


def _hipcc(sources, out, extra=(), verbose=False):
    """Compiles each source to an object in parallel, then links the shared library."""
    objdir = os.path.join(LIBDIR, "obj")
    os.makedirs(objdir, exist_ok=True)
    stem = os.path.splitext(os.path.basename(out))[0]
    objs = [os.path.join(objdir, f"{stem}.{os.path.basename(s)}.o") for s in sources]
    with ThreadPoolExecutor(max_workers=_jobs()) as ex:
        list(ex.map(lambda so: _run([HIPCC, *HIP_FLAGS, "-c", so[0], "-o", so[1]], verbose), zip(sources, objs)))
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, *extra, "-o", tmp], verbose)
    os.replace(tmp, out)


def build(verbose: bool = False) -> str:
    """Builds libbusfill.so (the product) and libbusfill_bench.so (the bench
    host's timed loops, linked against the product through its C-ABI)."""
    os.makedirs(LIBDIR, exist_ok=True)
    _hipcc([os.path.join(CSRC, s) for s in SOURCES], LIB, verbose=verbose)
    _hipcc([os.path.join(HERE, "host", "bench_host.hip")], BENCH_LIB,
           extra=["-L", LIBDIR, "-lbusfill", "-Wl,-rpath,$ORIGIN"], verbose=verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
