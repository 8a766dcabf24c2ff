"""Writes the committed golden fixtures of the oracle tests.

The reference holds no golden vectors for this path (its only GEMM
known-answer test is the macOS Accelerate check tests/test_mps_ops.py:24-41,
which compares against NumPy at runtime), so these fixtures are computed
here independently of NumPy's BLAS:

  tiny_gemm.npz        ragged tiny GEMMs (NN and NT, each input dtype) with
                       C computed by Python triple loops in math.fsum
                       (exactly rounded sums of fp64 products)
  tiny_linear.npz      tiny linear layers with bias and SiLU / GELU-tanh
                       epilogues evaluated with the math module, per element
  tiny_backward.npz    tiny linear-layer gradients (grad_input = g W,
                       grad_weight = g^T x, grad_bias = column sums of g)
                       by triple loops / column loops in math.fsum
  config_inputs.json   shape, dtype and SHA-256 of every generated input of
                       BASELINE.json's five configs (oracle.configs), so the
                       generators are pinned across machines

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import configs as cfg  # noqa: E402
from oracle.quant import quantize  # noqa: E402

TINY_SHAPES = [(1, 1, 1), (3, 5, 7), (4, 3, 2), (2, 9, 16), (5, 4, 33), (7, 6, 24)]
DTYPES = ["float32", "float16", "bfloat16"]


def fsum_matmul(a, b):
    m, k = a.shape
    n = b.shape[1]
    out = np.empty((m, n), np.float64)
    for i in range(m):
        for j in range(n):
            out[i, j] = math.fsum(float(a[i, p]) * float(b[p, j]) for p in range(k))
    return out


def silu(v):
    return v / (1.0 + math.exp(-v)) if v > -700 else 0.0


def gelu(v):
    return 0.5 * v * (1.0 + math.tanh(math.sqrt(2.0 / math.pi) * (v + 0.044715 * v ** 3)))


def tiny_gemm():
    rng = np.random.default_rng(20261201)
    arrays = {}
    for dt in DTYPES:
        for (m, n, k) in TINY_SHAPES:
            a = quantize(rng.uniform(-2, 2, (m, k)).astype(np.float32), dt)
            b = quantize(rng.uniform(-2, 2, (k, n)).astype(np.float32), dt)
            key = "%s_%dx%dx%d" % (dt, m, n, k)
            arrays[key + "_a"] = a
            arrays[key + "_b"] = b             # K x N
            arrays[key + "_c"] = fsum_matmul(a, b)
    np.savez(os.path.join(HERE, "tiny_gemm.npz"), **arrays)


def tiny_linear():
    rng = np.random.default_rng(7)
    arrays = {}
    for dt in DTYPES:
        for (m, n, k) in [(3, 5, 7), (2, 4, 16)]:
            x = quantize(rng.uniform(-3, 3, (m, k)).astype(np.float32), dt)
            w = quantize(rng.uniform(-1, 1, (n, k)).astype(np.float32), dt)
            b = quantize(rng.uniform(-1, 1, (n,)).astype(np.float32), dt)
            pre = fsum_matmul(x, w.T) + b.astype(np.float64)
            key = "%s_%dx%dx%d" % (dt, m, n, k)
            arrays[key + "_x"] = x
            arrays[key + "_w"] = w
            arrays[key + "_b"] = b
            arrays[key + "_bias"] = pre
            arrays[key + "_silu"] = np.vectorize(silu)(pre)
            arrays[key + "_gelu"] = np.vectorize(gelu)(pre)
    np.savez(os.path.join(HERE, "tiny_linear.npz"), **arrays)


def tiny_backward():
    rng = np.random.default_rng(793)
    arrays = {}
    for dt in DTYPES:
        for (m, n, k) in [(1, 3, 2), (5, 4, 7), (9, 6, 16), (3, 8, 5)]:
            g = quantize(rng.uniform(-2, 2, (m, n)).astype(np.float32), dt)
            x = quantize(rng.uniform(-2, 2, (m, k)).astype(np.float32), dt)
            w = quantize(rng.uniform(-1, 1, (n, k)).astype(np.float32), dt)
            key = "%s_%dx%dx%d" % (dt, m, n, k)
            arrays[key + "_g"] = g
            arrays[key + "_x"] = x
            arrays[key + "_w"] = w
            arrays[key + "_dx"] = fsum_matmul(g, w)
            gt = np.ascontiguousarray(g.T)
            arrays[key + "_dw"] = fsum_matmul(gt, x)
            arrays[key + "_db"] = np.array([math.fsum(float(g[i, j]) for i in range(m)) for j in range(n)])
    np.savez(os.path.join(HERE, "tiny_backward.npz"), **arrays)


def digest(a: np.ndarray) -> dict:
    a = np.ascontiguousarray(a, dtype=np.float32)
    return {"shape": list(a.shape), "sha256": hashlib.sha256(a.tobytes()).hexdigest(),
            "first": [float(v) for v in a.reshape(-1)[:4]]}


def config_inputs():
    out = {}
    c1 = cfg.c1_linear()
    out["C1"] = {"x": digest(c1.x), "w": digest(c1.w), "b": digest(c1.b)}
    a, b = cfg.c2_matmul(1024)
    out["C2_1024"] = {"a": digest(a), "b": digest(b)}
    for m in (1, 16):
        c3 = cfg.c3_linear(m)
        out["C3_M%d" % m] = {"x": digest(c3.x), "w": digest(c3.w), "b": digest(c3.b)}
    q, k, v, _ = cfg.c4_attention()
    out["C4"] = {"q": digest(q), "k": digest(k), "v": digest(v)}
    c5 = cfg.c5_projection("out")
    out["C5_out"] = {"x": digest(c5.x), "w": digest(c5.w), "b": digest(c5.b)}
    with open(os.path.join(HERE, "config_inputs.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    tiny_gemm()
    tiny_linear()
    tiny_backward()
    config_inputs()
    print("fixtures written to", HERE)
