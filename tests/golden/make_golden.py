"""Writes tests/golden/golden.npz: small seeded inputs for each weight format
with the oracle's fp16 dequant and fp64 dequantize-then-matmul outputs.

The reference ships no golden vectors for this path (it has no tests at all);
these fixtures freeze the oracle's answers so that any machine, compiler or
later change that alters them is caught, and give the GPU tests a stored
expected answer.  Their correctness rests on the known-answer and exhaustive
checks in tests/test_oracle.py.

Usage: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle as O  # noqa: E402

CASES = [  # (name, qtype, N, K, M, seed)
    ("planes", O.Q4_0_PLANES, 24, 512, 3, 11),
    ("q4_0", O.Q4_0, 24, 512, 3, 12),
    ("q4_k", O.Q4_K, 24, 512, 3, 13),
    ("q4_k_wide", O.Q4_K, 16, 1024, 17, 14),
]


def build():
    out = {}
    for name, qt, N, K, M, seed in CASES:
        w = O.gen_weights(qt, N, K, seed=seed)
        A = O.gen_act(M, K, seed=seed + 100)
        out[f"{name}/meta"] = np.array([qt, N, K, M, seed], np.int64)
        out[f"{name}/W"] = w.W
        if w.W_aux is not None:
            out[f"{name}/W_aux"] = w.W_aux
        out[f"{name}/A"] = A
        out[f"{name}/deq_f16"] = O.dequant_f16(w)
        out[f"{name}/C_f64"] = O.gemm_f64(w, A)
    return out


if __name__ == "__main__":
    path = os.path.join(HERE, "golden.npz")
    np.savez_compressed(path, **build())
    print(path, os.path.getsize(path), "bytes")
