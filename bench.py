#!/usr/bin/env python3
"""Benchmark of the batched int4-block GEMM on one MI355X.

Default run (the headline metric): Q4_K weights, N = K = 5120, batch M = 1, 8
and 32.  A step is one pass over a rotation of >= 1 GB of distinct weight
matrices already resident in HBM (72 matrices of 14.7 MB at 5120^2, so the
256 MB Infinity Cache cannot serve them): one GEMM per matrix.  Timing is
hipEvents recorded on the launch stream around exactly --steps passes (after
--warmup untimed ones); the timed GEMMs continue the rotation where the warmup
stopped, so no timed GEMM finds its matrix in a cache.  Before a rotation's
first timed configuration, about 0.1 s of untimed passes let the GPU's clocks
settle under load (`preheat_s` in the record).  The GEMMs are issued
back to back by the C++ bench host (bus-fill_amd/host/bench_host.hip) through
the libbusfill C-ABI.

Prints ONE JSON line.  `value` is the weight-stream GB/s at M = 1
(N*K*9/16 bytes / time per GEMM); `per_batch` carries M = 8 and 32; `roofline`
prices the algorithmic bytes (weights + A + C) per launch against the 8 TB/s
HBM peak, over the per-launch time committed in profiles/kernel_time.json (the
same event timing from a recorded run of this command), with this run's own
figures beside it (`*_events`); `cpu_baseline` is the oracle's CPU dequantize-then-matmul timed on
this host on a bounded sample of the same workload.  Two floors measured in the
same run stand beside them: `same_bytes_read_per_launch` (a plain streaming
read of one matrix's bytes per launch over the rotation, best of a few grids)
and `empty_kernel_per_launch` (back-to-back launches of a kernel that touches no
memory: the stream's per-kernel dispatch-and-completion cost).

Other workloads (--workload): q4_0 (18-byte blocks), planes (the reference
layout), layer (one 27B-class decoder layer's Q4_K linears at M = 32), sweep
(M = 1..128 on 5120x17408 and 17408x5120) and ggml (the ggml mul_mat hook).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "bus-fill_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "weight-stream HBM GB/s + tok/s, Q4_K 5120x5120 GEMM at batch 1/8/32"
HBM_PEAK_GBPS = 8000.0           # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0    # MI355X dense fp16 MFMA
ROTATION_BYTES = 1_050_000_000   # >= 1 GB of distinct weights per timing loop

QT = {"q4_k": 2, "q4_0": 0, "planes": 1}
QT_DESC = {"q4_k": "llama.cpp block_q4_K (144 B / 256 weights)",
           "q4_0": "llama.cpp block_q4_0 (18 B / 32 weights)",
           "planes": "reference planes Wq[N][K/2] u8 + Ws[N][K/32] fp16"}
SCALE_RANGE = {"q4_k": (0.001, 0.01), "q4_0": (0.002, 0.02), "planes": (0.002, 0.02)}

LAYER = [("qkv", 7168, 5120), ("o", 5120, 5120), ("gate", 17408, 5120), ("up", 17408, 5120), ("down", 5120, 17408)]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ device data
def row_layout(fmt, N, K):
    """Bytes of one matrix's row of the rotation buffer, and where its parts
    lie in it: (row bytes, W offset, W bytes, aux offset, aux bytes).  Every
    format keeps a whole matrix in one row, so a read of one matrix's bytes
    from its row start never leaves the row (the planes layout holds the code
    plane Wq[N][K/2] and then the scale plane Ws[N][K/32])."""
    wbytes = N * K * 9 // 16
    if fmt == "planes":
        return wbytes, 0, N * K // 2, N * K // 2, N * K // 16
    return wbytes, 0, wbytes, None, 0


class Rotation:
    """`count` distinct N x K matrices of one format in one device allocation,
    one matrix per row (row_layout)."""

    def __init__(self, fmt, N, K, min_bytes, seed, dev, scales=None, count=None):
        import torch
        self.fmt, self.N, self.K = fmt, N, K
        self.wbytes = N * K * 9 // 16
        self.count = count or max(1, math.ceil(min_bytes / self.wbytes))
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        lo, hi = scales or SCALE_RANGE[fmt]
        if fmt == "planes":
            row, w0, wn, a0, an = row_layout(fmt, N, K)
            self.buf = torch.randint(0, 256, (self.count, row), dtype=torch.uint8, device=dev, generator=g)
            self.W = self.buf[:, w0:w0 + wn]
            d = torch.rand((self.count, an // 2), device=dev, generator=g) * (hi - lo) + lo
            self.aux = self.buf[:, a0:a0 + an].view(torch.float16)
            self.aux.copy_(d.half())
        else:
            blk = 144 if fmt == "q4_k" else 18
            nblk = N * K // (256 if fmt == "q4_k" else 32)
            self.W = torch.randint(0, 256, (self.count, nblk * blk), dtype=torch.uint8, device=dev, generator=g)
            v = self.W.view(self.count * nblk, blk)
            nd = 2 if fmt == "q4_k" else 1          # d (and dmin for Q4_K)
            d = (torch.rand((self.count * nblk, nd), device=dev, generator=g) * (hi - lo) + lo).half()
            v[:, 0:2 * nd] = d.view(torch.uint8).view(self.count * nblk, 2 * nd)
            self.aux = None
            self.buf = self.W
        torch.cuda.synchronize()
        assert self.buf.shape == (self.count, self.wbytes) and self.buf.is_contiguous()

    @property
    def total_bytes(self):
        return self.count * self.wbytes

    def ptr_arrays(self):
        W = (ctypes.c_void_p * self.count)(*[self.W[i].data_ptr() for i in range(self.count)])
        aux = None
        if self.aux is not None:
            aux = (ctypes.c_void_p * self.count)(*[self.aux[i].data_ptr() for i in range(self.count)])
        return W, aux


def bench_lib():
    import busfill
    busfill.lib()                                  # the product library first (fails loudly)
    path = os.path.join(os.path.dirname(busfill.LIB_PATH), "libbusfill_bench.so")
    L = ctypes.CDLL(path)
    vp, i, d = ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_double)
    L.bfb_time_gemms.argtypes = [i, vp, vp, i, vp, i, vp, i, i, i, i, i, i, i, i, i, vp, d]
    L.bfb_time_sequence.argtypes = [i, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i, i, i, i, i, vp, d]
    L.bfb_time_sequence_batched.argtypes = [i, i, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i, i, i, i, vp, d]
    L.bfb_read_peak.argtypes = [vp, ctypes.c_size_t, i, vp, vp, d]
    L.bfb_read_slices.argtypes = [vp, i, ctypes.c_size_t, i, i, i, i, vp, vp, d]
    L.bfb_time_swiglu.argtypes = [i, vp, vp, i, vp, i, vp, vp, i, i, i, i, i, i, vp, d]
    L.bfb_copy.argtypes = [vp, vp, ctypes.c_size_t, i, vp, d]
    L.bfb_time_q8.argtypes = [i, vp, vp, i, vp, vp, vp, i, i, i, i, i, i, vp, d]
    L.bfb_time_ffn.argtypes = [i, vp, vp, vp, vp, vp, vp, i, vp, vp, vp, i, i, i, i, i, i, i, i, vp, d]
    L.bfb_time_ggml.argtypes = [i, vp, i, vp, vp, vp, i, i, i, i, i, i, vp, d]
    L.bfb_empty_launches.argtypes = [i, i, i, i, vp, vp, d]
    L.bfb_last_error.restype = ctypes.c_char_p
    for f in ("bfb_time_gemms", "bfb_time_sequence", "bfb_time_sequence_batched", "bfb_read_peak", "bfb_read_slices",
              "bfb_copy", "bfb_time_swiglu", "bfb_time_q8", "bfb_time_ffn", "bfb_time_ggml",
              "bfb_empty_launches"):
        getattr(L, f).restype = i
    return L


def P(arr):
    """A ctypes array (or None) as a plain pointer argument."""
    return None if arr is None else ctypes.cast(arr, ctypes.c_void_p)


_STREAM = None


def stream_handle():
    """A dedicated (default-priority) stream: the legacy null stream cannot be
    captured into a HIP graph."""
    global _STREAM
    import torch
    if _STREAM is None:
        _STREAM = torch.cuda.Stream()
    return _STREAM.cuda_stream


def time_gemm(L, rot, M, steps, warmup, graph, algo, dev, seed=7):
    """ms for steps * rot.count GEMMs (steps passes over the rotation) after
    warmup passes."""
    import torch
    torch.manual_seed(seed)
    A = torch.randn((M, rot.K), device=dev).half()
    C = torch.empty((M, rot.N), device=dev, dtype=torch.float32)
    W, aux = rot.ptr_arrays()
    ms = ctypes.c_double()
    torch.cuda.synchronize()
    rc = L.bfb_time_gemms(QT[rot.fmt], P(W), P(aux), rot.count, A.data_ptr(), rot.K, C.data_ptr(), rot.N, 0,
                          M, rot.N, rot.K, algo, warmup * rot.count, steps * rot.count, int(graph), stream_handle(),
                          ctypes.byref(ms))
    torch.cuda.synchronize()
    if rc != 0:
        raise RuntimeError("bench host: " + L.bfb_last_error().decode())
    if not torch.isfinite(C).all():
        raise RuntimeError("non-finite GEMM output during timing")
    return ms.value


PREHEAT_S = 0.1   # untimed work before a workload's first timed configuration


def preheat(L, rot, M, args, dev):
    """About PREHEAT_S seconds of untimed passes of the first configuration
    before anything of a rotation is timed: the GPU raises its clocks under
    sustained load, and without this the first configuration timed in a run
    measured 2-7 % slower than the same configuration timed later in it."""
    ms = time_gemm(L, rot, M, 1, 0, 0, args.algo_id, dev)
    passes = max(1, min(2000, int(math.ceil(PREHEAT_S * 1e3 / max(ms, 1e-3)))))
    time_gemm(L, rot, M, passes, 0, 0, args.algo_id, dev)


def gemm_record(rot, M, ms, steps, graph):
    """Per-GEMM figures from ms for `steps` passes over the rotation."""
    t = ms / 1e3 / (steps * rot.count)
    alg = rot.wbytes + M * rot.K * 2 + M * rot.N * 4
    flops = 2.0 * M * rot.N * rot.K
    return {
        "M": M, "us_per_gemm": round(t * 1e6, 4), "ms_per_pass": round(t * rot.count * 1e3, 5),
        "gemms_timed": steps * rot.count,
        "weight_GBps": round(rot.wbytes / t / 1e9, 2),
        "tok_s": round(M / t, 1),
        "alg_GBps": round(alg / t / 1e9, 2),
        "hbm_frac": round(alg / t / 1e9 / HBM_PEAK_GBPS, 4),
        "mfma_frac": round(flops / t / 1e12 / MFMA_F16_PEAK_TFLOPS, 5),
        "launch": "graph" if graph else "stream",
    }


def read_peak(L, rot):
    import torch
    sink = torch.zeros(1, dtype=torch.int32, device=rot.buf.device)
    ms = ctypes.c_double()
    nbytes = rot.buf.numel()
    rc = L.bfb_read_peak(rot.buf.data_ptr(), nbytes, 5, sink.data_ptr(), stream_handle(), ctypes.byref(ms))
    if rc != 0:
        raise RuntimeError("bench host: " + L.bfb_last_error().decode())
    return 5 * nbytes / (ms.value / 1e3) / 1e9


READ_GRIDS = ((256, 1024), (512, 512), (1024, 256), (2048, 256), (4096, 256))


def read_floor(L, rot, steps, warmup):
    """A plain streaming read of one matrix's bytes per launch, cycling through
    the rotation like the GEMM: the time a launch of that size needs to read
    its bytes with no other work (best of a few grid shapes)."""
    import torch
    sink = torch.zeros(1, dtype=torch.int32, device=rot.buf.device)
    rows = (ctypes.c_void_p * rot.count)(*[rot.buf[i].data_ptr() for i in range(rot.count)])
    nbytes = rot.wbytes // 16 * 16
    assert nbytes <= rot.buf.shape[1], "the read of one matrix must stay inside its row"
    best_us, best_grid = None, None
    for blocks, threads in READ_GRIDS:
        ms = ctypes.c_double()
        rc = L.bfb_read_slices(P(rows), rot.count, nbytes, blocks, threads, warmup * rot.count,
                               steps * rot.count, sink.data_ptr(), stream_handle(), ctypes.byref(ms))
        if rc != 0:
            raise RuntimeError("bench host: " + L.bfb_last_error().decode())
        us = ms.value * 1e3 / (steps * rot.count)
        if best_us is None or us < best_us:
            best_us, best_grid = us, (blocks, threads)
    return {"us_per_launch": round(best_us, 4), "GBps": round(rot.wbytes / (best_us / 1e6) / 1e9, 1),
            "bytes": rot.wbytes, "grid": list(best_grid)}


def empty_launch(L, steps):
    """Back-to-back launches of a kernel that touches no memory, with the
    batch-1 GEMM's grid (256 x 1024): the per-launch floor of any kernel on
    the stream (dispatch and completion), below which no GEMM launch goes."""
    import torch
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    ms = ctypes.c_double()
    rc = L.bfb_empty_launches(256, 1024, 200, steps, sink.data_ptr(), stream_handle(), ctypes.byref(ms))
    if rc != 0:
        raise RuntimeError("bench host: " + L.bfb_last_error().decode())
    return {"us_per_launch": round(ms.value * 1e3 / steps, 4), "grid": [256, 1024]}


# ------------------------------------------------------------------ CPU baseline
def cpu_threads():
    """Host threads for the CPU baseline: every CPU this process may run on,
    capped by OMP_NUM_THREADS when the environment sets it (the CPU share a job
    is granted on a shared host).  Returns (threads, cpus in the affinity mask,
    the OMP_NUM_THREADS text or None)."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS")
    n = min(avail, int(cap)) if cap and cap.isdigit() and int(cap) > 0 else avail
    return max(1, n), avail, cap


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(fmt, N, K, M, seconds):
    """The oracle's CPU dequantize-then-matmul (full fp32 dequant of W, then an
    fp32-accumulated matmul), timed on this host.  Only this leg of bench.py
    touches the oracle."""
    import numpy as np
    import oracle as O
    qt = {"q4_k": O.Q4_K, "q4_0": O.Q4_0, "planes": O.Q4_0_PLANES}[fmt]
    w = O.gen_weights(qt, N, K, seed=2024)
    A = O.gen_act(M, K, seed=2025)
    scratch = np.empty(N * K, np.float32)
    out = {}
    nthreads, avail, cap = cpu_threads()
    for label, threads, budget in (("all", nthreads, seconds), ("one", 1, max(2.0, seconds / 3))):
        O.cpu_dequant_matmul(w, A, threads=threads, scratch=scratch)          # warm
        n, tdq, tmm = 0, 0.0, 0.0
        t0 = time.perf_counter()
        while True:
            _, a, b = O.cpu_dequant_matmul(w, A, threads=threads, scratch=scratch)
            n, tdq, tmm = n + 1, tdq + a, tmm + b
            el = time.perf_counter() - t0
            if el >= budget:
                break
        t = el / n
        out[label] = {"threads": threads, "calls": n, "seconds": round(el, 2), "ms_per_call": round(t * 1e3, 3),
                      "ms_dequant": round(tdq / n * 1e3, 3), "ms_matmul": round(tmm / n * 1e3, 3),
                      "weight_GBps": round(N * K * 9 / 16 / t / 1e9, 4), "tok_s": round(M / t, 2)}
    a = out["all"]
    return {"value": a["weight_GBps"], "unit": "GB/s", "cores": a["threads"], "kind": "port",
            "sample": (f"{fmt} N={N} K={K} M={M}: {a['calls']} dequantize-then-matmul calls in "
                       f"{a['seconds']} s on {a['threads']} threads ({cpu_model()})"),
            "tok_s": a["tok_s"], "ms_per_call": a["ms_per_call"], "ms_dequant": a["ms_dequant"],
            "ms_matmul": a["ms_matmul"], "one_thread": out["one"],
            "host_cpus": os.cpu_count(), "affinity_cpus": avail, "omp_num_threads": cap, "cpu_model": cpu_model()}


def traffic_from_profiles(key):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        return json.load(open(path)).get(key)
    except (OSError, ValueError):
        return None


KERNEL_TIME = os.path.join("profiles", "kernel_time.json")


def kernel_time_from_profiles(key):
    """The committed per-launch time of one configuration (an entry that
    --kernel-time-out wrote), or None."""
    try:
        e = json.load(open(os.path.join(ROOT, KERNEL_TIME))).get(key)
    except (OSError, ValueError):
        return None
    return e if isinstance(e, dict) and e.get("us_per_launch", 0) > 0 else None


def library_digest():
    """The first 16 hex digits of the SHA-256 of libbusfill.so ("" if it
    cannot be read: every entry then starts over)."""
    import hashlib
    import busfill
    try:
        with open(busfill.LIB_PATH, "rb") as f:
            return hashlib.sha256(f.read()).hexdigest()[:16]
    except OSError:
        return ""


def write_kernel_time(path, fmt, N, K, recs, batches, argv):
    """Merges this run's per-launch times (the best launch mode of each batch
    size: HIP events around the timed passes, divided by the GEMMs timed) into
    the JSON file at path, one entry per configuration.  An entry written by a
    run of the same library build (the same SHA-256 of libbusfill.so) keeps
    the best of the runs and counts them (boxes differ by a few percent from
    one run to the next); a new build starts the entry over."""
    try:
        data = json.load(open(path))
    except (OSError, ValueError):
        data = {}
    lib = library_digest()
    for M in batches:
        r = best(recs, M)
        key = f"{fmt}_{N}_m{M}" if N == K else f"{fmt}_{N}x{K}_m{M}"
        old = data.get(key)
        same = bool(lib) and isinstance(old, dict) and old.get("lib_sha16") == lib
        runs = old.get("runs", 1) + 1 if same else 1
        if same and old.get("us_per_launch", 1e30) <= r["us_per_gemm"]:
            old["runs"] = runs
            continue
        data[key] = {
            "us_per_launch": r["us_per_gemm"], "launch": r["launch"], "gemms_timed": r["gemms_timed"],
            "ms_per_pass": r["ms_per_pass"], "lib_sha16": lib, "runs": runs,
            "how": "HIP events on the launch stream around the timed passes, / GEMMs timed; the best of the "
                   "runs of this library build",
            "command": "python3 bench.py " + " ".join(argv)}
    with open(path, "w") as f:
        json.dump(data, f, indent=1, sort_keys=True)
        f.write("\n")


# ------------------------------------------------------------------ workloads
def run_gemm_workload(L, fmt, N, K, batches, args, dev):
    rot = Rotation(fmt, N, K, ROTATION_BYTES, seed=11, dev=dev)
    log(f"[bench] {fmt} N={N} K={K}: {rot.count} matrices, {rot.total_bytes / 1e9:.3f} GB rotation")
    preheat(L, rot, batches[0], args, dev)
    recs = []
    for M in batches:
        for graph in ((0, 1) if args.graph == "both" else (int(args.graph),)):
            ms = time_gemm(L, rot, M, args.steps, args.warmup, graph, args.algo_id, dev)
            r = gemm_record(rot, M, ms, args.steps, graph)
            log(f"[bench] {fmt} M={M:3d} {r['launch']:6s}: {r['us_per_gemm']:8.3f} us  "
                f"{r['weight_GBps']:8.1f} GB/s  {r['tok_s']:10.0f} tok/s  hbm {r['hbm_frac']:.3f}")
            recs.append(r)
    peak = read_peak(L, rot)
    log(f"[bench] streaming-read over the rotation buffer: {peak:.1f} GB/s")
    rot.floor = read_floor(L, rot, args.steps, args.warmup)
    log(f"[bench] streaming-read of one matrix's {rot.wbytes} bytes per launch: {rot.floor['us_per_launch']:.3f} us "
        f"({rot.floor['GBps']:.1f} GB/s, grid {rot.floor['grid']})")
    return rot, recs, peak


def best(recs, M):
    c = [r for r in recs if r["M"] == M]
    return min(c, key=lambda r: r["us_per_gemm"])


def run_layer(L, args, dev):
    import torch
    M = args.layer_m
    layer_bytes = sum(n * k * 9 // 16 for _, n, k in LAYER)
    nl = max(1, math.ceil(ROTATION_BYTES / layer_bytes))
    log(f"[bench] layer: {nl} distinct layers x {layer_bytes / 1e6:.1f} MB")
    keep, seq = [], []
    for li in range(nl):
        for name, n, k in LAYER:
            rot = Rotation("q4_k", n, k, 1, seed=100 + 10 * li + len(seq), dev=dev)
            A = torch.randn((M, k), device=dev).half()
            C = torch.empty((M, n), device=dev)
            keep += [rot, A, C]
            seq.append((rot.W[0].data_ptr(), A.data_ptr(), C.data_ptr(), n, k))
    cnt = len(seq)
    arr = lambda t, xs: P((t * cnt)(*xs))
    ms = ctypes.c_double()
    nlin = len(LAYER)
    steps, warmup = args.steps * cnt, args.warmup * cnt      # passes over the nl layers, in GEMMs
    common = (arr(ctypes.c_int, [2] * cnt), arr(ctypes.c_void_p, [s[0] for s in seq]), None,
              arr(ctypes.c_void_p, [s[1] for s in seq]), arr(ctypes.c_int, [s[4] for s in seq]),
              arr(ctypes.c_void_p, [s[2] for s in seq]), arr(ctypes.c_int, [s[3] for s in seq]),
              arr(ctypes.c_int, [M] * cnt), arr(ctypes.c_int, [s[3] for s in seq]),
              arr(ctypes.c_int, [s[4] for s in seq]), 0)
    out = []
    # "single": one bf_gemm per linear; "batched": the layer's five linears in one
    # bf_gemm_batched call (one launch per kernel the linears take)
    modes = ("single", "batched") if args.layer_launch == "both" else (args.layer_launch,)
    for mode in modes:
        for graph in ((0, 1) if args.graph == "both" else (int(args.graph),)):
            torch.cuda.synchronize()
            if mode == "single":
                rc = L.bfb_time_sequence(cnt, *common, args.algo_id, warmup, steps, graph, stream_handle(),
                                         ctypes.byref(ms))
            else:
                rc = L.bfb_time_sequence_batched(cnt, nlin, *common, warmup, steps, graph, stream_handle(),
                                                 ctypes.byref(ms))
            torch.cuda.synchronize()
            if rc != 0:
                raise RuntimeError("bench host: " + L.bfb_last_error().decode())
            t_layer = ms.value / 1e3 / (steps / nlin)
            pass_ms = ms.value / args.steps
            rec = {"M": M, "us_per_layer": round(t_layer * 1e6, 3), "layer_tok_s": round(M / t_layer, 1),
                   "weight_GBps": round(layer_bytes / t_layer / 1e9, 2),
                   "hbm_frac": round(layer_bytes / t_layer / 1e9 / HBM_PEAK_GBPS, 4),
                   "launch": "graph" if graph else "stream", "calls": mode, "layers_rotated": nl,
                   "ms_per_pass": round(pass_ms, 5), "gemms_timed": steps}
            log(f"[bench] layer M={M} {mode} {rec['launch']}: {rec['us_per_layer']:.2f} us/layer "
                f"{rec['weight_GBps']:.1f} GB/s {rec['layer_tok_s']:.0f} tok/s")
            out.append(rec)
    return out


COPY_BYTES = 256 << 20


def run_copy(L, args, dev):
    """The calibration kernel for the HBM byte counters: a 128-bit copy of
    exactly COPY_BYTES (read COPY_BYTES, write COPY_BYTES per launch)."""
    import torch
    src = torch.randint(0, 256, (COPY_BYTES,), dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    reps = max(1, min(args.steps, 50))
    ms = ctypes.c_double()
    torch.cuda.synchronize()
    rc = L.bfb_copy(src.data_ptr(), dst.data_ptr(), COPY_BYTES, reps, stream_handle(), ctypes.byref(ms))
    torch.cuda.synchronize()
    if rc != 0:
        raise RuntimeError("bench host: " + L.bfb_last_error().decode())
    if not torch.equal(src, dst):
        raise RuntimeError("copy kernel produced a wrong copy")
    t = ms.value / 1e3 / reps
    return {"metric": "HBM copy GB/s (read + write), calibration kernel", "value": round(2 * COPY_BYTES / t / 1e9, 1),
            "unit": "GB/s", "n_gpus": 1, "steps": reps, "warmup": 0, "ms_per_step": round(t * 1e3, 6),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8", "data": "synthetic",
            "config": {"workload": f"k_stream_copy of {COPY_BYTES} bytes", "bytes_read": COPY_BYTES,
                       "bytes_written": COPY_BYTES}}


def run_swiglu(L, args, dev):
    """The down projection of a 27B-class SwiGLU block (K = 17408 -> N = 5120)
    fed by the gate|up output: SiLU*up fused into the GEMM's activation load
    against bf_swiglu_f16 + bf_gemm (two launches and an fp16 intermediate)."""
    import torch
    N, K = 5120, 17408
    rot = Rotation("q4_k", N, K, ROTATION_BYTES, seed=N, dev=dev)
    W, aux = rot.ptr_arrays()
    res = []
    for M in (1, 2):
        gu = torch.randn((M, 2 * K), device=dev).half()
        a = torch.empty((M, K), device=dev, dtype=torch.float16)
        C = torch.empty((M, N), device=dev, dtype=torch.float32)
        r = {"M": M, "N": N, "K": K, "calls_per_pass": rot.count}
        for fused in (1, 0):
            ms = ctypes.c_double()
            torch.cuda.synchronize()
            rc = L.bfb_time_swiglu(QT["q4_k"], P(W), P(aux), rot.count, gu.data_ptr(), 2 * K, a.data_ptr(),
                                   C.data_ptr(), M, N, K, fused, args.warmup * rot.count, args.steps * rot.count,
                                   stream_handle(), ctypes.byref(ms))
            torch.cuda.synchronize()
            if rc != 0:
                raise RuntimeError("bench host: " + L.bfb_last_error().decode())
            r["fused_us" if fused else "unfused_us"] = round(ms.value * 1e3 / (args.steps * rot.count), 3)
        log(f"[bench] swiglu down projection M={M}: fused {r['fused_us']:.2f} us, "
            f"swiglu + gemm {r['unfused_us']:.2f} us")
        res.append(r)
    return res


FFN_FORMS = {"one_launch": 1, "two_launches": 2, "calls": 3}


def run_ffn(L, args, dev):
    """The 27B-class SwiGLU feed-forward block (gate and up 5120 -> 17408,
    SiLU(g) * u, down 17408 -> 5120; 150.4 MB of Q4_K weights) through
    bf_ffn_swiglu_ex in each form that serves the batch, over a >= 1 GB
    rotation of distinct blocks.  Q4_K scales d, dmin ~ U[1e-4, 1e-3]: with
    the single-GEMM workloads' U[1e-3, 1e-2] the weights' mean is near 1 and
    SiLU(g) * u overflows fp16."""
    import torch
    K, F, N = 5120, 17408, 5120
    sr = (1e-4, 1e-3)
    block = 3 * F * K * 9 // 16
    count = max(1, math.ceil(ROTATION_BYTES / block))
    rots = [Rotation("q4_k", F, K, 0, seed=1, dev=dev, scales=sr, count=count),
            Rotation("q4_k", F, K, 0, seed=2, dev=dev, scales=sr, count=count),
            Rotation("q4_k", N, F, 0, seed=3, dev=dev, scales=sr, count=count)]
    ptrs = [r.ptr_arrays()[0] for r in rots]
    log(f"[bench] ffn: {count} distinct blocks x {block / 1e6:.1f} MB")
    res = []
    for M in [int(x) for x in (args.batches or "1,2,8,32").split(",")]:
        A = torch.randn((M, K), device=dev).half()
        gu = torch.empty((M, 2 * F), device=dev, dtype=torch.float16)
        C = torch.empty((M, N), device=dev, dtype=torch.float32)
        for form, fid in FFN_FORMS.items():
            if fid != FFN_FORMS["calls"] and M > 2:
                continue
            for graph in ((0, 1) if args.graph == "both" else (int(args.graph),)):
                ms = ctypes.c_double()
                torch.cuda.synchronize()
                rc = L.bfb_time_ffn(QT["q4_k"], P(ptrs[0]), None, P(ptrs[1]), None, P(ptrs[2]), None, count,
                                    A.data_ptr(), gu.data_ptr(), C.data_ptr(), M, K, F, N, fid,
                                    args.warmup * count, args.steps * count, graph, stream_handle(),
                                    ctypes.byref(ms))
                torch.cuda.synchronize()
                if rc != 0:
                    raise RuntimeError("bench host: " + L.bfb_last_error().decode())
                if not torch.isfinite(C).all():
                    raise RuntimeError("non-finite feed-forward output during timing")
                t = ms.value / 1e3 / (args.steps * count)
                r = {"M": M, "form": form, "launch": "graph" if graph else "stream",
                     "us_per_block": round(t * 1e6, 3), "weight_GBps": round(block / t / 1e9, 2),
                     "tok_s": round(M / t, 1), "blocks_timed": args.steps * count}
                log(f"[bench] ffn M={M} {form} {r['launch']}: {r['us_per_block']:.2f} us/block "
                    f"{r['weight_GBps']:.1f} GB/s")
                res.append(r)
    return res, count, block


def run_q8(L, args, dev):
    """The integer-dot activation path (int8 activations per 32 values,
    v_dot4_i32_i8) against the fp16 GEMM, Q4_K 5120x5120, M = 1-16: the q8
    GEMM alone, and quantize + GEMM per call."""
    import torch
    N = K = 5120
    rot = Rotation("q4_k", N, K, ROTATION_BYTES, seed=N, dev=dev)
    W, aux = rot.ptr_arrays()
    res = []
    for M in (1, 2, 4, 8, 16):
        A = torch.randn((M, K), device=dev).half()
        Aq = torch.empty((M * K + 8 * M * (K // 32),), device=dev, dtype=torch.uint8)
        C = torch.empty((M, N), device=dev, dtype=torch.float32)
        r = {"M": M, "N": N, "K": K, "calls_per_pass": rot.count}
        for mode, key in ((0, "fp16_us"), (2, "q8_gemm_us"), (1, "q8_quant_gemm_us")):
            ms = ctypes.c_double()
            torch.cuda.synchronize()
            rc = L.bfb_time_q8(QT["q4_k"], P(W), P(aux), rot.count, A.data_ptr(), Aq.data_ptr(), C.data_ptr(),
                               M, N, K, mode, args.warmup * rot.count, args.steps * rot.count, stream_handle(),
                               ctypes.byref(ms))
            torch.cuda.synchronize()
            if rc != 0:
                raise RuntimeError("bench host: " + L.bfb_last_error().decode())
            r[key] = round(ms.value * 1e3 / (args.steps * rot.count), 3)
        log(f"[bench] q8 path M={M:2d}: fp16 GEMM {r['fp16_us']:.2f} us, q8 GEMM {r['q8_gemm_us']:.2f} us, "
            f"quantize + q8 GEMM {r['q8_quant_gemm_us']:.2f} us")
        res.append(r)
    return res


def run_ggml(L, args, dev):
    """The ggml mul_mat hook on the default GEMM (Q4_K 5120x5120 over the
    rotation): bf_ggml_mul_mat with F32 src1 (at M = 1 rounded by the batch-1
    kernel as it loads the row, otherwise staged to fp16 by a launch of its
    own) and with F16 src1 (read in place), against bf_gemm on the fp16 rows."""
    import torch
    N = K = 5120
    rot = Rotation("q4_k", N, K, ROTATION_BYTES, seed=N, dev=dev)
    W, _ = rot.ptr_arrays()
    res = []
    for M in [int(x) for x in (args.batches or "1,8,32").split(",")]:
        A32 = torch.randn((M, K), device=dev)
        A16 = A32.half()
        C = torch.empty((M, N), device=dev, dtype=torch.float32)
        r = {"M": M, "N": N, "K": K, "calls_per_pass": rot.count}
        for mode, key in ((0, "bf_gemm_us"), (2, "ggml_f16_us"), (1, "ggml_f32_us")):
            ms = ctypes.c_double()
            torch.cuda.synchronize()
            rc = L.bfb_time_ggml(QT["q4_k"], P(W), rot.count, A32.data_ptr(), A16.data_ptr(), C.data_ptr(), M, N, K,
                                 mode, args.warmup * rot.count, args.steps * rot.count, stream_handle(),
                                 ctypes.byref(ms))
            torch.cuda.synchronize()
            if rc != 0:
                raise RuntimeError("bench host: " + L.bfb_last_error().decode())
            r[key] = round(ms.value * 1e3 / (args.steps * rot.count), 3)
        log(f"[bench] ggml hook M={M:2d}: bf_gemm {r['bf_gemm_us']:.2f} us, F16 src1 {r['ggml_f16_us']:.2f} us, "
            f"F32 src1 {r['ggml_f32_us']:.2f} us")
        res.append(r)
    return res


SWEEP_SHAPES = "17408x5120,5120x17408"
SWEEP_BATCHES = "1,2,3,4,6,8,16,32,64,128"


def run_sweep(L, args, dev):
    res = []
    shapes = [tuple(int(v) for v in s.split("x")) for s in (args.shapes or SWEEP_SHAPES).split(",")]
    for (N, K) in shapes:
        rot = Rotation("q4_k", N, K, ROTATION_BYTES, seed=N, dev=dev)
        batches = [int(x) for x in (args.batches or SWEEP_BATCHES).split(",")]
        preheat(L, rot, batches[0], args, dev)
        for M in batches:
            ms = time_gemm(L, rot, M, args.steps, args.warmup, int(args.graph == "1"), args.algo_id, dev)
            r = gemm_record(rot, M, ms, args.steps, args.graph == "1")
            r.update({"N": N, "K": K})
            log(f"[bench] sweep N={N} K={K} M={M:3d}: {r['us_per_gemm']:8.2f} us {r['weight_GBps']:8.1f} GB/s "
                f"mfma {r['mfma_frac']:.4f}")
            res.append(r)
        del rot
    return res


# ------------------------------------------------------------------ kernel traces
def kernel_key(name):
    """A dispatch's kernel name without its argument list (template arguments
    kept): the text before the parenthesis that matches the final one."""
    name = name.strip()
    if name.startswith("void "):
        name = name[5:]
    if not name.endswith(")"):
        return name
    depth = 0
    for i in range(len(name) - 1, -1, -1):
        depth += {")": 1, "(": -1}.get(name[i], 0)
        if depth == 0:
            return name[:i]
    return name


def trace_summary(path, per_pass, labels):
    """Per-launch kernel durations from a `rocprofv3 --kernel-trace` CSV.

    The library's dispatches (kernel names in namespace bf) are taken in start
    order and grouped into runs of consecutive dispatches of one kernel; each
    run is cut into passes of `per_pass` dispatches (one pass over the weight
    rotation).  For each run: the mean and median dispatch duration (end -
    start of each dispatch), and over its passes the median and minimum of
    (last end - first start) / per_pass, the time per launch with the gaps
    between launches included -- the figure comparable to HIP events around
    back-to-back launches.  `labels` names the runs in order."""
    import csv
    import statistics as st
    rows = [r for r in csv.DictReader(open(path)) if "bf::" in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    runs = []
    for r in rows:
        k = kernel_key(r["Kernel_Name"])
        if runs and runs[-1][0] == k:
            runs[-1][1].append(r)
        else:
            runs.append((k, [r]))
    runs = [(k, rs) for k, rs in runs if len(rs) >= per_pass]
    out = {}
    for i, (k, rs) in enumerate(runs):
        d = [int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in rs]
        spans = [(int(rs[j + per_pass - 1]["End_Timestamp"]) - int(rs[j]["Start_Timestamp"])) / per_pass
                 for j in range(0, len(rs) - per_pass + 1, per_pass)]
        gaps = [int(b["Start_Timestamp"]) - int(a["End_Timestamp"]) for a, b in zip(rs, rs[1:])]
        label = labels[i] if i < len(labels) else f"run{i}"
        out[label] = {"kernel": k, "dispatches": len(rs), "passes": len(spans), "per_pass": per_pass,
                      "us_dispatch_mean": round(st.mean(d) / 1e3, 4), "us_dispatch_median": round(st.median(d) / 1e3, 4),
                      "us_span_per_launch_median": round(st.median(spans) / 1e3, 4),
                      "us_span_per_launch_min": round(min(spans) / 1e3, 4),
                      "us_gap_median": round(st.median(gaps) / 1e3, 4) if gaps else 0.0}
    return out


def roofline_record(key, alg_bytes, t_live):
    """The roofline of the dominant kernel: algorithmic bytes per launch over
    the per-launch time committed in profiles/kernel_time.json for this
    configuration (the basis of `frac`), beside the same figures from this
    run's HIP events (`*_events`).  Without a committed entry the basis is this
    run's time, and `duration_source` says so."""
    kt = kernel_time_from_profiles(key)
    t = kt["us_per_launch"] / 1e6 if kt else t_live
    return {"bound": "hbm", "achieved": round(alg_bytes / t / 1e9, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(alg_bytes / t / 1e9 / HBM_PEAK_GBPS, 4),
            "traffic": traffic_from_profiles(key),
            "algorithmic_bytes_per_launch": alg_bytes,
            "us_per_launch": round(t * 1e6, 4),
            "duration_source": f"{KERNEL_TIME} [{key}]" if kt else "this run's HIP events",
            "us_per_launch_events": round(t_live * 1e6, 4),
            "achieved_events": round(alg_bytes / t_live / 1e9, 2),
            "frac_events": round(alg_bytes / t_live / 1e9 / HBM_PEAK_GBPS, 4)}


def counter_summary(path):
    """Per-dispatch means of the counters in a `rocprofv3 --pmc` CSV, per
    kernel of this library (namespace bf) and the bench's own kernels: each
    dispatch's Counter_Value summed over the rows it has for one counter, then
    averaged over the kernel's dispatches."""
    import csv
    import statistics as st
    per = {}
    for r in csv.DictReader(open(path)):
        name = kernel_key(r["Kernel_Name"])
        if "bf::" not in r["Kernel_Name"] and "k_stream" not in name:
            continue
        d = per.setdefault(name, {}).setdefault(r["Counter_Name"], {})
        d[r["Dispatch_Id"]] = d.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
    out = {}
    for name, counters in per.items():
        out[name] = {"dispatches": max(len(v) for v in counters.values())}
        for c, v in sorted(counters.items()):
            out[name][c] = round(st.mean(v.values()), 2)
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30,
                    help="timed passes over the >= 1 GB weight rotation per configuration (one GEMM per matrix)")
    ap.add_argument("--warmup", type=int, default=3, help="untimed passes before the timed ones")
    ap.add_argument("--workload", default="q4_k",
                    choices=["q4_k", "q4_0", "planes", "layer", "sweep", "copy", "swiglu", "q8", "ffn", "ggml"])
    ap.add_argument("--batches", default=None,
                    help="batch rows M to time (default 1,8,32; sweep: " + SWEEP_BATCHES + ")")
    ap.add_argument("--shapes", default=None,
                    help="sweep workload: NxK weight shapes (default " + SWEEP_SHAPES + ")")
    ap.add_argument("--graph", default="both", choices=["0", "1", "both"],
                    help="issue launches on the stream (0), replay a HIP graph (1), or time both")
    ap.add_argument("--layer-m", type=int, default=32, help="layer workload: batch rows (config: 32)")
    ap.add_argument("--layer-launch", default="both", choices=["single", "batched", "both"],
                    help="layer workload: one bf_gemm per linear, one bf_gemm_batched per layer, or both")
    ap.add_argument("--algo", default="auto",
                    choices=["auto", "mfma", "dot2", "simple", "lds", "slab", "split", "dense"])
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--out", default=None, help="also write the full record to this JSON file")
    ap.add_argument("--kernel-time-out", default=None, metavar="JSON",
                    help="q4_k / q4_0 / planes: merge this run's per-launch times (one entry per batch size) into "
                         "this JSON file (" + KERNEL_TIME + " is the roofline's committed basis)")
    ap.add_argument("--trace-summary", default=None, metavar="CSV",
                    help="no GPU work: summarize a rocprofv3 kernel-trace CSV of an earlier bench run "
                         "(per-launch durations per run of one kernel) as one JSON line")
    ap.add_argument("--counter-summary", default=None, metavar="CSV",
                    help="no GPU work: per-dispatch counter means per kernel of a rocprofv3 --pmc CSV, as one JSON "
                         "line")
    ap.add_argument("--trace-labels", default="q4_k_5120_m1,q4_k_5120_m8,q4_k_5120_m32",
                    help="--trace-summary: names of the runs, in order")
    ap.add_argument("--trace-pass", type=int, default=72, help="--trace-summary: dispatches per pass")
    args = ap.parse_args()
    if args.trace_summary or args.counter_summary:
        rec = (trace_summary(args.trace_summary, args.trace_pass, args.trace_labels.split(","))
               if args.trace_summary else counter_summary(args.counter_summary))
        line = json.dumps(rec)
        if args.out:
            with open(args.out, "w") as f:
                f.write(line + "\n")
        print(line, flush=True)
        return
    args.algo_id = {"auto": 0, "mfma": 1, "dot2": 2, "simple": 3, "lds": 4, "slab": 5, "split": 6,
                    "dense": 7}[args.algo]

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the GEMM runs on a single MI355X and there is no "
              "multi-GPU path (sharding would split N across GPUs, one independent GEMM each); "
              "run it with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    dev = torch.device("cuda:0")
    L = bench_lib()
    batches = [int(x) for x in (args.batches if args.workload != "sweep" and args.batches else "1,8,32").split(",")]

    if args.workload in ("q4_k", "q4_0", "planes"):
        fmt = args.workload
        rot, recs, peak = run_gemm_workload(L, fmt, 5120, 5120, batches, args, dev)
        head = best(recs, batches[0])
        t = head["us_per_gemm"] / 1e6
        alg_bytes = rot.wbytes + head["M"] * rot.K * 2 + head["M"] * rot.N * 4
        record = {
            "metric": METRIC if fmt == "q4_k" else METRIC.replace("Q4_K", fmt.upper()),
            "value": head["weight_GBps"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": head["ms_per_pass"],
            "preheat_s": PREHEAT_S,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
            "data": "synthetic",
            "config": {"workload": f"{fmt} GEMM N=K=5120, batch M={head['M']} (per_batch: M={batches})",
                       "format": QT_DESC[fmt], "N": 5120, "K": 5120, "batches": batches,
                       "rotation_matrices": rot.count, "rotation_bytes": rot.total_bytes,
                       "launch": head["launch"], "accumulate": "fp32", "algo": args.algo},
            "tok_s": head["tok_s"], "us_per_gemm": head["us_per_gemm"],
            "step": (f"one pass over the rotation: {rot.count} GEMMs, one per distinct matrix, "
                     f"{rot.total_bytes} weight bytes"),
            "gemms_timed": head["gemms_timed"], "weight_bytes_timed": head["gemms_timed"] * rot.wbytes,
            "per_batch": [best(recs, M) for M in batches],
            "all_runs": recs,
            "hbm_read_measured_GBps": round(peak, 1),
            "same_bytes_read_per_launch": rot.floor,
            "empty_kernel_per_launch": empty_launch(L, 2000),
            "roofline": roofline_record(f"{fmt}_5120_m{head['M']}", alg_bytes, t),
        }
        if args.kernel_time_out:
            write_kernel_time(args.kernel_time_out, fmt, 5120, 5120, recs, batches, sys.argv[1:])
        del rot
        torch.cuda.empty_cache()
        if not args.no_cpu:
            log("[bench] CPU baseline ...")
            record["cpu_baseline"] = cpu_baseline(fmt, 5120, 5120, batches[0], args.cpu_seconds)
            # the reference's CPU-runnable case: Q4_0 blocks, M = 1, the same path
            c0 = cpu_baseline("q4_0", 5120, 5120, 1, args.cpu_seconds / 2)
            record["cpu_baseline"]["q4_0_m1"] = {k: c0[k] for k in ("value", "unit", "cores", "sample", "tok_s",
                                                                    "ms_per_call", "ms_dequant", "ms_matmul",
                                                                    "one_thread")}
    elif args.workload == "layer":
        recs = run_layer(L, args, dev)
        b = min(recs, key=lambda r: r["us_per_layer"])
        record = {"metric": "layer-sum weight-stream GB/s + tok/s, 27B-class decoder layer Q4_K linears at batch "
                            f"{args.layer_m}",
                  "value": b["weight_GBps"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
                  "warmup": args.warmup, "ms_per_step": b["ms_per_pass"],
                  "step": f"one pass over {b['layers_rotated']} distinct layers ({len(LAYER)} GEMMs each)",
                  "us_per_layer": b["us_per_layer"],
                  "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
                  "data": "synthetic",
                  "config": {"workload": "q4_k qkv 5120->7168, o 5120->5120, gate/up 5120->17408, down 17408->5120",
                             "M": args.layer_m, "launch": b["launch"], "calls": b["calls"]},
                  "layer_tok_s": b["layer_tok_s"], "runs": recs}
    elif args.workload == "copy":
        record = run_copy(L, args, dev)
    elif args.workload == "swiglu":
        recs = run_swiglu(L, args, dev)
        head = recs[0]
        record = {"metric": "down projection with SiLU*up (Q4_K 17408->5120): us per call, fused vs swiglu + gemm",
                  "value": head["fused_us"], "unit": "us", "n_gpus": 1, "steps": args.steps,
                  "warmup": args.warmup, "ms_per_step": round(head["fused_us"] * head["calls_per_pass"] / 1e3, 6),
                  "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
                  "data": "synthetic",
                  "config": {"workload": "q4_k down projection N=5120 K=17408 fed by gate|up [M][2K], M=1 and 2"},
                  "runs": recs}
    elif args.workload == "ffn":
        recs, count, block = run_ffn(L, args, dev)
        head = min((r for r in recs if r["M"] == recs[0]["M"]), key=lambda r: r["us_per_block"])
        record = {"metric": "SwiGLU feed-forward block (Q4_K gate/up 5120->17408, down 17408->5120): "
                            "weight-stream GB/s and us per block",
                  "value": head["weight_GBps"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
                  "warmup": args.warmup, "ms_per_step": round(head["us_per_block"] * count / 1e3, 6),
                  "step": f"one pass over {count} distinct blocks ({block} weight bytes each)",
                  "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
                  "data": "synthetic",
                  "config": {"workload": "q4_k SwiGLU block K=5120 F=17408 N=5120", "M": head["M"],
                             "form": head["form"], "launch": head["launch"]},
                  "runs": recs}
    elif args.workload == "q8":
        recs = run_q8(L, args, dev)
        head = next(r for r in recs if r["M"] == 8)
        record = {"metric": "integer-dot (int8 activation) path vs fp16 GEMM, Q4_K 5120x5120: us per GEMM",
                  "value": head["q8_gemm_us"], "unit": "us", "n_gpus": 1, "steps": args.steps,
                  "warmup": args.warmup, "ms_per_step": round(head["q8_gemm_us"] * head["calls_per_pass"] / 1e3, 6),
                  "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
                  "data": "synthetic",
                  "config": {"workload": "q4_k N=5120 K=5120, M=1-16, value at M=8"}, "runs": recs}
    elif args.workload == "ggml":
        recs = run_ggml(L, args, dev)
        head = recs[0]
        record = {"metric": "ggml mul_mat hook, Q4_K 5120x5120, F32 src1: us per call",
                  "value": head["ggml_f32_us"], "unit": "us", "n_gpus": 1, "steps": args.steps,
                  "warmup": args.warmup, "ms_per_step": round(head["ggml_f32_us"] * head["calls_per_pass"] / 1e3, 6),
                  "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
                  "data": "synthetic",
                  "config": {"workload": f"q4_k N=5120 K=5120 through bf_ggml_mul_mat, value at M={head['M']}"},
                  "runs": recs}
    else:
        recs = run_sweep(L, args, dev)
        record = {"metric": "Q4_K GEMM batch sweep: weight-stream GB/s and MFMA utilisation",
                  "value": max(r["weight_GBps"] for r in recs), "unit": "GB/s", "n_gpus": 1,
                  "steps": args.steps, "warmup": args.warmup, "higher_is_better": True, "scaling": "weak",
                  "vs_baseline": None, "dtype": "f16", "data": "synthetic",
                  "config": {"workload": f"q4_k M in {args.batches or SWEEP_BATCHES} on "
                                         f"{args.shapes or SWEEP_SHAPES}", "algo": args.algo},
                  "sweep": recs}
    line = json.dumps(record)
    if args.out:
        with open(args.out, "w") as f:
            f.write(line + "\n")
    print(line, flush=True)


if __name__ == "__main__":
    main()
