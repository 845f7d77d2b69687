"""Per-workgroup timelines of the GEMM kernels: a copy of the library whose
kernel stamps s_memrealtime (100 MHz) at fixed points into a device array,
one row of 256 stamps per workgroup.

    python bus-fill_amd/devtools/timeline.py build lds|dense|split     (CPU: patch and compile)
    python bus-fill_amd/devtools/timeline.py run lds|dense|split N K M (GPU: 60 GEMMs over a 1 GB
                                                                         rotation, the last one's stamps)

`build` writes bus-fill_amd/devtools/_tl_<kernel>/ (libbusfill.so with the
stamps and bf_tl_copy); `run` loads that copy instead of the product library
and prints medians over the workgroups, in microseconds from the first
workgroup's start.  Stamps:

lds (k_gemm_lds; the batch-1 form records its reductions):
    127 workgroup start (wave 0); 64 + g: loader 0 has issued its step of
    group g; e < 64: the wave that took step e has seen its data (marker set);
    224 + t / 232 + t: the reducer of sub-tile t < 8 starts / ends waiting for
    its steps; 240 + t: sub-tile t stored.
dense (k_gemm_dense):
    127 workgroup start; compute wave 0: u / 40 + u start / end of its wait for
    activation half-slab u, 128 + v / 168 + v for weight unit v; 80 + u / 208 + v
    activation / weight loader issuing unit u / v; 121 compute wave 0 done.
split (k_gemm_split, one launch):
    127 workgroup start; 64 + i: loader 0 issuing unit i; 125 loader 0's loads
    landed; i / 32 + i: compute wave 0 starts / ends its wait for unit i; 120 the
    last compute wave done with its units, 121 compute wave 0 done; 122 tile 0's
    sums stored (issued); 123 the last split (reducer) starts reading the
    partials, 124 its wave 0 has written its share of C.
"""
from __future__ import annotations

import importlib.util
import os
import shutil
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)

# the stamp is an ordered instruction (asm volatile, waited for), so the
# compiler keeps it where it stands
HEADER = ("namespace bf {\n__device__ uint64_t g_tl[8192 * 256];\n"
          "__device__ __forceinline__ uint64_t tl_now() {\n"
          "    uint64_t t;\n"
          "    asm volatile(\"s_memrealtime %0\\n\\ts_waitcnt lgkmcnt(0)\" : \"=s\"(t) :: \"memory\");\n"
          "    return t;\n}\n"
          "namespace {\n"
          "#define TL(k) do { if (lane == 0 && blockIdx.x < 8192 && (k) < 256) "
          "g_tl[(size_t)blockIdx.x * 256 + (k)] = tl_now(); } while (0)\n")
EXPORT = ('extern "C" int bf_tl_copy(void* host, size_t bytes) {\n'
          '    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(bf::g_tl), bytes, 0, hipMemcpyDeviceToHost);\n}\n'
          # a one-wave kernel that stamps row 8191, column k: launched before and after
          # a GEMM on the same stream, it brackets the GEMM's dispatch
          'namespace bf {\n__global__ void k_tl_mark(int k) {\n'
          '    const uint64_t t = tl_now();\n'
          '    if (threadIdx.x == 0) g_tl[(size_t)8191 * 256 + k] = t;\n}\n}  // namespace bf\n'
          'extern "C" int bf_tl_mark(int k) {\n'
          '    hipLaunchKernelGGL(bf::k_tl_mark, dim3(1), dim3(64), 0, (hipStream_t)0, k);\n'
          '    return (int)hipGetLastError();\n}\n')

# (old, new) replacements, each of which must match exactly once
PATCHES = {
    "lds": ("bf_gemm_lds.hip", [
        ("namespace bf {\nnamespace {\n", HEADER),
        ("    const int tile0 = bid * nsub;\n", "    const int tile0 = bid * nsub;\n    if (wave == 0) TL(127);\n"),
        ("            if (g4 == 0) clear_flags_and_meet();\n",
         "            if (j == 0 && g4 < 32) TL(64 + g4);\n            if (g4 == 0) clear_flags_and_meet();\n"),
        ("            // the step's slot is free again (its reads have completed)\n",
         "            if (e < 64) TL(e);\n            // the step's slot is free again (its reads have completed)\n"),
        ("            // a wave's LDS operations complete in order: the slot is free once this\n",
         "            if (e < 64) TL(e);\n            // a wave's LDS operations complete in order: the slot is free once this\n"),
        ("            wait_count(&flags[kSubCount + t_in], nsteps, flags + kPoison);\n",
         "            if (t_in < 8) TL(224 + t_in);\n            wait_count(&flags[kSubCount + t_in], nsteps, flags + kPoison);\n"
         "            if (t_in < 8) TL(232 + t_in);\n"),
        ("                if (g == 0 && kg == 0 && mt < M && row < N) store_c(mt, row, y);\n            }\n",
         "                if (g == 0 && kg == 0 && mt < M && row < N) store_c(mt, row, y);\n            }\n"
         "            if (t_in < 8) TL(240 + t_in);\n"),
    ]),
    "dense": ("bf_gemm_dense.hip", [
        ("namespace bf {\nnamespace {\n", HEADER),
        ("    const int nsg = K >> 8;\n    const int t0 = range_first(p, T, G), t1 = range_first(p + 1, T, G);\n",
         "    const int nsg = K >> 8;\n    const int t0 = range_first(p, T, G), t1 = range_first(p + 1, T, G);\n"
         "    if (wave == 0) TL(127);\n"),
        ("                wait_flags(flags + kDnAReady + kDnNLA * u, kDnNLA, lane, flags + kDnPoison);\n",
         "                if (c == 0 && u < 40) TL(u);\n"
         "                wait_flags(flags + kDnAReady + kDnNLA * u, kDnNLA, lane, flags + kDnPoison);\n"
         "                if (c == 0 && u < 40) TL(40 + u);\n"),
        ("                    const uint32_t off = 512u * (uint32_t)sg + 128u * (uint32_t)h;\n",
         "                    const uint32_t off = 512u * (uint32_t)sg + 128u * (uint32_t)h;\n"
         "                    if (ja == 0 && u < 40) TL(80 + u);\n"),
        ("            wait_flags(flags + kDnWReady + kDnNLW * v, kDnNLW, lane, flags + kDnPoison);\n",
         "            if (c == 0 && v < 40) TL(128 + v);\n"
         "            wait_flags(flags + kDnWReady + kDnNLW * v, kDnNLW, lane, flags + kDnPoison);\n"
         "            if (c == 0 && v < 40) TL(168 + v);\n"),
        ("                    const uint32_t wb = lds0 + (uint32_t)(kDnFlags + (v % DW) * kDnWSlot);\n",
         "                    const uint32_t wb = lds0 + (uint32_t)(kDnFlags + (v % DW) * kDnWSlot);\n"
         "                    if (j == 0 && v < 40) TL(208 + v);\n"),
        ("        t += s1 - s0;\n    }\n}\n\n// One workgroup per CU",
         "        t += s1 - s0;\n    }\n    if (c == 0) TL(121);\n}\n\n// One workgroup per CU"),
    ]),
    "split": ("bf_gemm_split.hip", [
        ("namespace bf {\nnamespace {\n", HEADER),
        ("    const int sg0 = s * nsgS;\n", "    const int sg0 = s * nsgS;\n    if (wave == 0) TL(127);\n"),
        ("            if (i == 0) clear_flags_and_meet();\n",
         "            if (j == 0 && i < 32) TL(64 + i);\n            if (i == 0) clear_flags_and_meet();\n"),
        ("        asm volatile(\"s_waitcnt vmcnt(0)\" ::: \"memory\");\n        return;\n    }\n",
         "        asm volatile(\"s_waitcnt vmcnt(0)\" ::: \"memory\");\n        if (j == 0) TL(125);\n        return;\n    }\n"),
        ("        wait_flags(flags + 16 + 4 * i, NL, lane, flags + kSpPoison);\n",
         "        if (c == 0 && i < 32) TL(i);\n        wait_flags(flags + 16 + 4 * i, NL, lane, flags + kSpPoison);\n"
         "        if (c == 0 && i < 32) TL(32 + i);\n"),
        ("    // the tile's first wave adds the others' sums (in wave order) and writes the tile\n",
         "    if (c == 0) TL(121);\n    if (c == NC - 1) TL(120);\n"
         "    // the tile's first wave adds the others' sums (in wave order) and writes the tile\n"),
        ("        if (SUM2) return;\n        if (!slots) {\n", "        if (c == 0) TL(122);\n        if (SUM2) return;\n        if (!slots) {\n"),
        ("        if (s != S - 1) return;\n", "        if (s != S - 1) return;\n        if (c == 0) TL(123);\n"),
        ("                else ((float*)C)[(int64_t)(m4 + i) * ldc + n0 + nl] = y;\n            }\n        }\n        return;\n",
         "                else ((float*)C)[(int64_t)(m4 + i) * ldc + n0 + nl] = y;\n            }\n        }\n"
         "        if (c == 0) TL(124);\n        return;\n"),
    ]),
}


def out_dir(kernel: str) -> str:
    return os.path.join(HERE, f"_tl_{kernel}")


def build(kernel: str) -> str:
    fname, patches = PATCHES[kernel]
    spec = importlib.util.spec_from_file_location("bf_build", os.path.join(PKG, "build.py"))
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    out = out_dir(kernel)
    src = os.path.join(out, "csrc")
    shutil.rmtree(out, ignore_errors=True)
    shutil.copytree(b.CSRC, src)
    path = os.path.join(src, fname)
    text = open(path).read()
    for old, new in patches:
        if text.count(old) != 1:
            raise SystemExit(f"{fname}: anchor found {text.count(old)} times: {old[:60]!r}")
        text = text.replace(old, new)
    text = text.rstrip()
    if not text.endswith("}  // namespace bf"):
        raise SystemExit(f"{fname}: does not end with the bf namespace")
    open(path, "w").write(text + "\n" + EXPORT)
    b.CSRC, b.LIBDIR = src, out
    b.HIP_FLAGS = [src if x == os.path.join(PKG, "csrc") else x for x in b.HIP_FLAGS]
    b._hipcc([os.path.join(src, s) for s in b.SOURCES], os.path.join(out, "libbusfill.so"))
    shutil.rmtree(os.path.join(out, "obj"), ignore_errors=True)
    shutil.rmtree(src)
    return out


def _pct(x, q):
    import numpy as np
    return float(np.percentile(x, q))


def run(kernel: str, N: int, K: int, M: int) -> None:
    import ctypes
    lib = os.path.join(out_dir(kernel), "libbusfill.so")
    if not os.path.exists(lib):
        raise SystemExit(f"{lib} is missing: run `timeline.py build {kernel}` first")
    os.environ["BUSFILL_LIBDIR"] = out_dir(kernel)
    sys.path[:0] = [ROOT, PKG]
    import numpy as np
    import torch
    import busfill as bf
    from bench import Rotation
    dev = torch.device("cuda:0")
    L = bf.lib()
    if os.path.realpath(L._name) != os.path.realpath(lib):
        raise SystemExit(f"loaded {L._name}, not the stamped copy")
    L.bf_tl_copy.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    rot = Rotation("q4_k", N, K, 1_050_000_000, seed=11, dev=dev)
    A = torch.randn((M, K), device=dev).half()
    C = torch.empty((M, N), device=dev)
    algo = {"dense": bf.ALGO_DENSE, "split": bf.ALGO_SPLIT}.get(kernel, bf.ALGO_LDS)
    for i in range(60):
        bf.gemm(bf.Q4_K, rot.W[i % rot.count], None, A, C, M, N, K, algo=algo)
    # the last GEMM bracketed by two one-wave stamp kernels on the same stream
    L.bf_tl_mark(0)
    bf.gemm(bf.Q4_K, rot.W[60 % rot.count], None, A, C, M, N, K, algo=algo)
    L.bf_tl_mark(1)
    torch.cuda.synchronize()
    h = np.zeros((8192, 256), np.uint64)
    if L.bf_tl_copy(h.ctypes.data, h.nbytes) != 0:
        raise SystemExit("bf_tl_copy failed")
    marks = h[8191, :2].astype(np.int64)
    h[8191, :] = 0
    used = h[:, 127] != 0
    hu = h[used]
    H = (hu.astype(np.int64) - int(hu[:, 127].min())) / 100.0

    def col(k):
        ok = hu[:, k] != 0
        return H[ok, k]

    print(f"{kernel} N={N} K={K} M={M}: {int(used.sum())} workgroups; starts median {np.median(H[:, 127]):.2f} "
          f"max {H[:, 127].max():.2f} us")
    if marks.all():
        last = int(hu[hu != 0].astype(np.int64).max())
        t0 = int(hu[:, 127].min())
        print(f"stamp kernel before -> first workgroup start: {(t0 - marks[0]) / 100.0:.2f} us; last stamp of the GEMM "
              f"-> stamp kernel after: {(marks[1] - last) / 100.0:.2f} us; before -> after: "
              f"{(marks[1] - marks[0]) / 100.0:.2f} us")
    if kernel == "lds":
        print("loader 0, step of group g issued (median us):",
              " ".join(f"{g}:{np.median(col(64 + g)):.2f}" for g in range(32) if (hu[:, 64 + g] != 0).any()))
        print(" step  data seen (median / p90 / max us)")
        for e in range(64):
            x = col(e)
            if len(x):
                print(f"  {e:3d}  {np.median(x):6.2f} {_pct(x, 90):6.2f} {x.max():6.2f}")
        for t in range(8):
            s, w, d = col(224 + t), col(232 + t), col(240 + t)
            if len(d):
                print(f" sub-tile {t}: reducer waits {np.median(s):.2f} -> {np.median(w):.2f}, stored "
                      f"{np.median(d):.2f} (p90 {_pct(d, 90):.2f}, max {d.max():.2f})")
        ends = np.max(np.where(hu[:, 240:248] != 0, H[:, 240:248], 0), axis=1)
        print(f"workgroup end (last of sub-tiles 0-7 stored): median {np.median(ends):.2f} p90 {_pct(ends, 90):.2f} "
              f"max {ends.max():.2f}")
    elif kernel == "split":
        print("loader 0, unit i issued (median us):",
              " ".join(f"{i}:{np.median(col(64 + i)):.2f}" for i in range(32) if (hu[:, 64 + i] != 0).any()))
        print(" unit  wait start  wait end   (compute wave 0, medians us)")
        for i in range(32):
            if not (hu[:, i] != 0).any():
                break
            print(f"  {i:3d}  {np.median(col(i)):9.2f}  {np.median(col(32 + i)):8.2f}")
        for k, what in ((125, "loader 0's loads landed"), (121, "compute wave 0 done"),
                        (120, "last compute wave done"), (122, "tile 0 sums stored"),
                        (123, "reducer starts reading"), (124, "reducer wave 0 wrote C")):
            x = col(k)
            if len(x):
                print(f"{what:>26}: median {np.median(x):6.2f} p90 {_pct(x, 90):6.2f} max {x.max():6.2f} "
                      f"({len(x)} workgroups)")
        ends = np.max(np.where(hu[:, 120:126] != 0, H[:, 120:126], 0), axis=1)
        print(f"workgroup end (last stamp): median {np.median(ends):.2f} p90 {_pct(ends, 90):.2f} max {ends.max():.2f}")
    else:
        d = col(121)
        print(f"compute done: median {np.median(d):.2f} p90 {_pct(d, 90):.2f} max {d.max():.2f}")
        print("  u  A issued  wait start  wait end   (medians, us)")
        for u in range(40):
            if not (hu[:, u] != 0).any():
                break
            print(f" {u:2d}  {np.median(col(80 + u)):7.2f}  {np.median(col(u)):9.2f}  {np.median(col(40 + u)):8.2f}")
        print("  v  W issued  wait start  wait end")
        for v in range(40):
            if not (hu[:, 128 + v] != 0).any():
                break
            print(f" {v:2d}  {np.median(col(208 + v)):7.2f}  {np.median(col(128 + v)):9.2f}  {np.median(col(168 + v)):8.2f}")


if __name__ == "__main__":
    if len(sys.argv) < 3 or sys.argv[1] not in ("build", "run") or sys.argv[2] not in PATCHES:
        raise SystemExit(__doc__)
    if sys.argv[1] == "build":
        print(build(sys.argv[2]))
    else:
        run(sys.argv[2], *(int(x) for x in sys.argv[3:6]))
