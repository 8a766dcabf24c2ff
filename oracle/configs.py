"""Seeded inputs, work counts and tolerances of BASELINE.json's five configs
(test infrastructure).

Generation rule (applies to every config): ``np.random.default_rng(seed)``,
draws in the order x -> W -> b (C4: Q -> K -> V), float32 draws, then
round-to-nearest-even to the config dtype.  The same quantized arrays feed
the device, the CPU baseline and the fp64 oracle.

Tolerances:
  fp32        normwise  max|y - y_cpu| / max|y_cpu| <= 1e-5 * sqrt(K)
  bf16/fp16   max|y - y_fp64| <= 2e-2 * sqrt(K / 1024)
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from .quant import quantize

PEAK_BF16_FLOPS = 2.5166e15   # dense bf16/fp16 MFMA, 256 CU x 4096 flop/clk x 2.4 GHz
PEAK_FP32_FLOPS = 157.3e12    # fp32 matrix
PEAK_HBM_BPS = 8.0e12         # HBM3E


def tol_fp32(k: int) -> float:
    return 1e-5 * math.sqrt(k)


def tol_16(k: int) -> float:
    return 2e-2 * math.sqrt(k / 1024.0)


def normwise_err(y, y_ref) -> float:
    y = np.asarray(y, np.float64)
    y_ref = np.asarray(y_ref, np.float64)
    denom = float(np.max(np.abs(y_ref)))
    return float(np.max(np.abs(y - y_ref))) / (denom if denom > 0 else 1.0)


def abs_err(y, y_ref) -> float:
    return float(np.max(np.abs(np.asarray(y, np.float64) - np.asarray(y_ref, np.float64))))


def gemm_flops(m: int, n: int, k: int, batch: int = 1) -> float:
    return 2.0 * m * n * k * batch


def gemm_bytes(m: int, n: int, k: int, in_size: int, out_size: int, batch: int = 1,
               bias: bool = False, b_batched: bool = True) -> float:
    """Compulsory HBM bytes: A and B read once, C written once, bias once."""
    a = batch * m * k * in_size
    b = (batch if b_batched else 1) * n * k * in_size
    c = batch * m * n * out_size
    return float(a + b + c + (n * in_size if bias else 0))


@dataclass
class LinearCase:
    name: str
    x: np.ndarray       # float32 values, already quantized to dtype
    w: np.ndarray
    b: np.ndarray | None
    dtype: str
    act: str | None


def _normal(rng, shape, std):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def c1_linear() -> LinearCase:
    """C1: nn.Linear fp32 x[64,512] @ W^T[512,512] + b; x, W ~ N(0,1)/sqrt(512),
    b ~ U(-0.1, 0.1), seed 0."""
    rng = np.random.default_rng(0)
    s = 1.0 / math.sqrt(512)
    x = _normal(rng, (64, 512), s)
    w = _normal(rng, (512, 512), s)
    b = rng.uniform(-0.1, 0.1, 512).astype(np.float32)
    return LinearCase("C1", x, w, b, "float32", None)


def c2_matmul(n: int):
    """C2: fp32 A[n,n] @ B[n,n], A, B ~ U(-1,1), seed 1."""
    rng = np.random.default_rng(1)
    a = rng.uniform(-1.0, 1.0, (n, n)).astype(np.float32)
    b = rng.uniform(-1.0, 1.0, (n, n)).astype(np.float32)
    return a, b


def c3_linear(m: int, k: int = 4096, n: int = 11008) -> LinearCase:
    """C3: bf16 x[M,4096] @ W^T[4096->11008] + b, SiLU; x ~ N(0,1),
    W ~ N(0,0.02), b ~ N(0,0.01), seed 2."""
    rng = np.random.default_rng(2)
    x = quantize(_normal(rng, (m, k), 1.0), "bfloat16")
    w = quantize(_normal(rng, (n, k), 0.02), "bfloat16")
    b = quantize(_normal(rng, (n,), 0.01), "bfloat16")
    return LinearCase("C3_M%d" % m, x, w, b, "bfloat16", "silu")


def c4_attention(bh: int = 60, s: int = 4096, d: int = 64):
    """C4: fp16 Q, K, V [60, 4096, 64] ~ N(0,1), seed 3; scale 1/sqrt(64)."""
    rng = np.random.default_rng(3)
    q = quantize(_normal(rng, (bh, s, d), 1.0), "float16")
    k = quantize(_normal(rng, (bh, s, d), 1.0), "float16")
    v = quantize(_normal(rng, (bh, s, d), 1.0), "float16")
    return q, k, v, 1.0 / math.sqrt(d)


C5_TOKENS = 13 * (60 * 90 // 4) + 226   # 17776
C5_PROJ = {
    # name: (K, N, bias, act)
    "qkv": (1920, 5760, False, None),
    "out": (1920, 1920, True, None),
    "mlp_up": (1920, 7680, True, "gelu_tanh"),
    "mlp_down": (7680, 1920, True, None),
}


def c5_projection(name: str, tokens: int = C5_TOKENS) -> LinearCase:
    """C5: bf16 CogVideoX-2B-style DiT projections; activations ~ N(0,1),
    weights ~ N(0,0.02), bias ~ N(0,0.01); seed 4 + index of the
    projection in (qkv, out, mlp_up, mlp_down)."""
    k, n, has_b, act = C5_PROJ[name]
    rng = np.random.default_rng(4 + list(C5_PROJ).index(name))
    x = quantize(_normal(rng, (tokens, k), 1.0), "bfloat16")
    w = quantize(_normal(rng, (n, k), 0.02), "bfloat16")
    b = quantize(_normal(rng, (n,), 0.01), "bfloat16") if has_b else None
    return LinearCase("C5_" + name, x, w, b, "bfloat16", act)
