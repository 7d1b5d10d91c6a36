"""Writes the committed golden fixtures under tests/golden/.

Run from the repo root:  python tests/golden/make_golden.py

1. reference_kats.npz -- the known-answer tests held by ZigNeuron's own test
   files, re-encoded as data (inputs exactly as the reference tests build
   them, expected outputs as the reference tests define them).  Integer-valued
   cases have exact expected outputs from int64 arithmetic.  The reference is
   Zig and cannot be run here; these values are read from the test sources.
2. oracle_cases.npz -- small seeded ragged cases for every layout / epilogue,
   with expected outputs produced by the oracle (oracle/liboracle.so).  They
   pin the oracle against drift (tests re-derive and compare bit-exactly) and
   give the GPU parity tests a fixed, committed expected output.

Inputs use numpy's PCG64 (np.random.default_rng(seed)); uniform values are
float32 draws in [0,1) mapped to [-1,1).
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle  # noqa: E402  (test infrastructure)


def f32(x):
    return np.asarray(x, dtype=np.float32)


def reference_kats() -> dict:
    kats = {}

    # src/test/unit/backend.zig:196-225 "backend matmul correctness"
    kats["correctness_a"] = f32([1, 2, 3, 4, 5, 6])
    kats["correctness_b"] = f32([7, 8, 9, 10, 11, 12])
    kats["correctness_c"] = f32([58, 64, 139, 154])
    kats["correctness_mnk"] = np.array([2, 2, 3], np.int64)

    # src/test/unit/backend.zig:227-250 "backend matmul large matrix": 64^3 ones -> 64
    kats["ones64_c"] = np.full(64 * 64, 64.0, np.float32)

    # src/test/unit/backend.zig:17-51 "backend matmul cpu": m=2,n=3,k=2,
    # a[i] = (i % 10) / 10, b[i] = ((i+1) % 10) / 10; the test checks c[0]
    # against its own sequential f32 dot product sum_p a[p]*b[p*n].
    m, n, k = 2, 3, 2
    a = f32([np.float32(i % 10) / np.float32(10.0) for i in range(m * k)])
    b = f32([np.float32((i + 1) % 10) / np.float32(10.0) for i in range(k * n)])
    exp0 = np.float32(0.0)
    for p in range(k):
        exp0 = np.float32(exp0 + np.float32(a[p] * b[p * n]))
    kats["cpu_small_a"], kats["cpu_small_b"] = a, b
    kats["cpu_small_c0"] = f32([exp0])
    kats["cpu_small_mnk"] = np.array([m, n, k], np.int64)

    # Integer-valued fixtures of src/cuda_matmul_validation.zig (exact in fp32:
    # every partial sum stays far below 2^24).  Expected = int64 matmul.
    def int_case(tag, m, n, k, fa, fb, line):
        ai = np.array([fa(i) for i in range(m * k)], np.int64)
        bi = np.array([fb(i) for i in range(k * n)], np.int64)
        ci = ai.reshape(m, k) @ bi.reshape(k, n)
        kats[f"{tag}_a"], kats[f"{tag}_b"] = ai.astype(np.float32), bi.astype(np.float32)
        kats[f"{tag}_c"] = ci.astype(np.float32).ravel()
        kats[f"{tag}_mnk"] = np.array([m, n, k], np.int64)
        kats[f"{tag}_src"] = np.array(line)

    int_case("small64", 64, 64, 64, lambda i: i % 10, lambda i: (i * 3) % 10,
             "src/cuda_matmul_validation.zig:20-49")
    int_case("medium256", 256, 256, 256, lambda i: i % 5, lambda i: (i * 2) % 5,
             "src/cuda_matmul_validation.zig:52-73")
    int_case("nonsquare", 128, 64, 256, lambda i: i % 7, lambda i: (i * 3) % 7,
             "src/cuda_matmul_validation.zig:76-97")
    # "cuda_matmul_accumulate" (:100-125): the second call accumulates, so C = 2*A*B.
    int_case("accum64", 64, 64, 64, lambda i: i % 3, lambda i: (i * 2) % 3,
             "src/cuda_matmul_validation.zig:100-125")

    # Dense layer KATs, src/test/unit/layer.zig (W [in x out], bias [out]).
    # forward relu (:16-33), negative input (:169-186), precision (:188-206),
    # bias contribution with .linear (:208-222):
    #   rows: act, w0, w1, bias, x0, x1, expected
    kats["dense_fwd_act"] = np.array(["relu", "relu", "relu", "linear"])
    kats["dense_fwd"] = f32([
        [1.0, 1.0, 0.0, 1.0, 1.0, 2.0],
        [1.0, 1.0, 0.0, -1.0, -1.0, 0.0],
        [1.2345678, 2.3456789, 0.9876543, 1.0, 1.0, 1.2345678 + 2.3456789 + 0.9876543],
        [0.0, 0.0, 5.0, 0.0, 0.0, 5.0],
    ])
    # backward relu (:35-55) and sigmoid (:224-241): activated_output given,
    # grad_output = 1; rows: act, w0, w1, x0, x1, y, gx0, gx1
    kats["dense_bwd_act"] = np.array(["relu", "sigmoid"])
    kats["dense_bwd"] = f32([
        [1.0, 1.0, 1.0, 1.0, 2.0, 1.0, 1.0],
        [0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0],
    ])

    # Activation KATs, src/test/unit/backend.zig:53-75 (relu on i/2-2.5),
    # :77-101 (sigmoid on i/2-1, output[2] = 0.5), :103-132 (sigmoid backward
    # = s*(1-s) with grad_output 1).
    kats["act_relu_x"] = f32([np.float32(i) / np.float32(2.0) - np.float32(2.5) for i in range(10)])
    kats["act_relu_y"] = np.maximum(kats["act_relu_x"], 0).astype(np.float32)
    kats["act_sigmoid_x"] = f32([np.float32(i) / np.float32(2.0) - np.float32(1.0) for i in range(5)])
    return kats


def uniform(rng, shape, lo=-1.0, hi=1.0):
    return (rng.random(shape, dtype=np.float32) * np.float32(hi - lo) + np.float32(lo)).astype(np.float32)


def oracle_cases() -> dict:
    """Seeded ragged cases; keys <name>_{a,b,bias,c0,c,meta}."""
    cases = {}
    specs = [
        # name, layout, m, n, k, accumulate, act, seed
        ("nn_ragged", "nn", 37, 45, 29, False, None, 1),
        ("nn_blocked", "nn", 67, 70, 97, False, None, 2),
        ("nn_acc", "nn", 33, 40, 65, True, None, 3),
        ("tn_ragged", "tn", 45, 37, 61, False, None, 4),
        ("tn_acc", "tn", 31, 66, 34, True, None, 5),
        ("nt_ragged", "nt", 29, 53, 47, False, None, 6),
        ("nt_acc", "nt", 64, 33, 96, True, None, 7),
        ("bias_lin", "nn", 40, 10, 128, False, "linear", 8),
        ("bias_relu", "nn", 48, 33, 79, False, "relu", 9),
        ("bias_sigmoid", "nn", 21, 30, 50, False, "sigmoid", 10),
        ("bias_tanh", "nn", 19, 35, 77, False, "tanh", 11),
        ("k1", "nn", 5, 7, 1, False, None, 12),
        ("m1", "nn", 1, 9, 13, False, None, 13),
    ]
    for name, layout, m, n, k, acc, act, seed in specs:
        rng = np.random.default_rng(seed)
        if layout == "tn":
            a = uniform(rng, (k, m))
        else:
            a = uniform(rng, (m, k))
        b = uniform(rng, (n, k)) if layout == "nt" else uniform(rng, (k, n))
        c0 = uniform(rng, (m, n))
        bias = uniform(rng, (n,))
        if act is not None:
            c = oracle.matmul_bias_act(a, b, bias, m, n, k, act)
        elif layout == "nn":
            c = oracle.matmul(a, b, m, n, k, accumulate=acc, c_init=c0)
        elif layout == "tn":
            c = oracle.matmul_tn(a, b, m, n, k, accumulate=acc, c_init=c0)
        else:
            c = oracle.matmul_nt(a, b, m, n, k, accumulate=acc, c_init=c0)
        cases[f"{name}_a"], cases[f"{name}_b"] = a, b
        cases[f"{name}_bias"], cases[f"{name}_c0"], cases[f"{name}_c"] = bias, c0, c
        cases[f"{name}_meta"] = np.array([layout, str(m), str(n), str(k), str(int(acc)), act or "none"])
    cases["names"] = np.array([s[0] for s in specs])
    return cases


def main() -> None:
    oracle.build()
    np.savez_compressed(os.path.join(HERE, "reference_kats.npz"), **reference_kats())
    np.savez_compressed(os.path.join(HERE, "oracle_cases.npz"), **oracle_cases())
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
