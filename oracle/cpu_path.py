"""The reference's Linux CPU path for the matmul hot path, restated in NumPy
(test infrastructure; never imported by the product path).

On Linux the reference computes every operation of this path with NumPy
(its Cython CPU kernels are built on macOS only, reference setup.py:319-333),
so the restatement below is the same sequence of NumPy calls:

  matmul        np.matmul(a, b)                       reference tensor.py:1516-1519
  matmul_nt     matmul(a, b.transpose(-2, -1))        reference tensor.py:1538-1539
  linear        x @ W.T (+ b)                         reference nn/layers.py:129-131
  F.linear      np.matmul(x, W.T) (+ b)               reference nn/functional.py:388-393
  silu          x * (1 / (1 + exp(-x)))               reference nn/functional.py:58-59
  gelu (tanh)   0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3)))
                                                      reference nn/functional.py:79-82
  softmax       e = exp(x - max); e / sum(e)          reference nn/functional.py:137-141
  sdpa          scores = q @ k^T; *= scale; += mask; softmax; @ v
                                                      reference nn/functional.py:323-357
  matmul_tn     np.matmul(a^T, b)                     reference autograd.py:296,813-818,
                                                      _mps_ops.pyx:279-298 (A^T @ B)
  linear_backward  g @ W, g_2d^T @ x_2d, sum(g_2d, 0) reference autograd.py:793-822
  sum_dim       np.sum(x, axis=dim)                   reference autograd.py:819;
                                                      shapes as _cuda_ops.pyx:1710-1741

The *_f64 functions are the closed forms in float64 on the (already
quantized) inputs: the accuracy oracle for every dtype.
"""
from __future__ import annotations

import math

import numpy as np

SQRT_2_OVER_PI = math.sqrt(2.0 / math.pi)
GELU_C = 0.044715


# ---------------------------------------------------------------- fp32 path

def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """reference tensor.py:1516-1519 (Linux CPU branch)."""
    return np.matmul(a, b)


def matmul_nt(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """reference tensor.py:1538-1539: matmul(a, b.transpose(-2, -1))."""
    return np.matmul(a, np.swapaxes(b, -2, -1))


def linear(x: np.ndarray, w: np.ndarray, b: np.ndarray | None = None) -> np.ndarray:
    """reference nn/layers.py:129-131: result = x @ W.T; result + bias."""
    y = x @ w.T
    if b is not None:
        y = y + b
    return y


def silu(x: np.ndarray) -> np.ndarray:
    """reference nn/functional.py:58-59."""
    sig = 1.0 / (1.0 + np.exp(-x))
    return x * sig


def gelu_tanh(x: np.ndarray) -> np.ndarray:
    """reference nn/functional.py:79-82."""
    return 0.5 * x * (1 + np.tanh(SQRT_2_OVER_PI * (x + GELU_C * x ** 3)))


def softmax(x: np.ndarray, axis: int = -1) -> np.ndarray:
    """reference nn/functional.py:137-141."""
    x_max = x.max(axis=axis, keepdims=True)
    e = np.exp(x - x_max)
    e_sum = e.sum(axis=axis, keepdims=True)
    np.divide(e, e_sum, out=e)
    return e


def sdpa(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float | None = None,
         attn_mask: np.ndarray | None = None) -> np.ndarray:
    """reference nn/functional.py:323-357 without dropout: the additive
    attn_mask is added to the scaled scores with NumPy broadcasting
    (:339-341) before the max-shifted softmax."""
    d = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    scores = np.matmul(q, np.swapaxes(k, -2, -1))
    scores *= scale
    if attn_mask is not None:
        scores += attn_mask
    s_max = scores.max(axis=-1, keepdims=True)
    scores -= s_max
    np.exp(scores, out=scores)
    s_sum = scores.sum(axis=-1, keepdims=True)
    np.divide(scores, s_sum, out=scores)
    return np.matmul(scores, v)


def matmul_tn(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """A^T @ B with A (..., K, M), B (..., K, N): reference autograd.py:296
    (np.matmul(a_T, g)) and :818 (np.matmul(g_2d.T, x_2d)); the macOS
    blas_sgemm_tn (_mps_ops.pyx:279-298) computes the same product."""
    return np.matmul(np.swapaxes(a, -2, -1), b)


def linear_backward(g: np.ndarray, x: np.ndarray, w: np.ndarray, has_bias: bool = True):
    """reference autograd.py:793-822, LinearBackward.backward, the NumPy
    branch (:816-821): grad_input = g @ W, grad_weight = g_2d.T @ x_2d,
    grad_bias = np.sum(g_2d, axis=0)."""
    g_2d = g.reshape(-1, g.shape[-1])
    x_2d = x.reshape(-1, x.shape[-1])
    grad_input = np.matmul(g, w)
    grad_weight = np.matmul(g_2d.T, x_2d)
    if has_bias:
        return grad_input, grad_weight, np.sum(g_2d, axis=0)
    return grad_input, grad_weight


def sum_dim(x: np.ndarray, dim: int = -1, keepdim: bool = False) -> np.ndarray:
    """np.sum over one axis (reference autograd.py:819); output shape as
    the reference's dev_sum_dim (_cuda_ops.pyx:1710-1741)."""
    return np.sum(x, axis=dim, keepdims=keepdim)


# ------------------------------------------------------- fp64 closed forms

def act_f64(y: np.ndarray, act: str | None) -> np.ndarray:
    if act in (None, "none"):
        return y
    if act == "silu":
        return y / (1.0 + np.exp(-y))
    if act in ("gelu", "gelu_tanh"):
        return 0.5 * y * (1.0 + np.tanh(SQRT_2_OVER_PI * (y + GELU_C * y ** 3)))
    raise ValueError(act)


def linear_f64(x, w, b=None, act: str | None = None, alpha: float = 1.0) -> np.ndarray:
    """act(alpha * x . W^T + b) in float64."""
    y = alpha * (np.asarray(x, np.float64) @ np.asarray(w, np.float64).T)
    if b is not None:
        y = y + np.asarray(b, np.float64)
    return act_f64(y, act)


def matmul_f64(a, b) -> np.ndarray:
    return np.matmul(np.asarray(a, np.float64), np.asarray(b, np.float64))


def linear_backward_f64(g, x, w):
    """(g @ W, g_2d^T @ x_2d, column sums of g_2d) in float64."""
    g64 = np.asarray(g, np.float64)
    g_2d = g64.reshape(-1, g64.shape[-1])
    x_2d = np.asarray(x, np.float64).reshape(-1, np.shape(x)[-1])
    return g64 @ np.asarray(w, np.float64), g_2d.T @ x_2d, g_2d.sum(axis=0)


def softmax_f64(x, scale: float = 1.0) -> np.ndarray:
    s = np.asarray(x, np.float64) * scale
    s = s - s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    return e / e.sum(axis=-1, keepdims=True)


def sdpa_f64(q, k, v, scale: float, attn_mask=None) -> np.ndarray:
    s = np.matmul(np.asarray(q, np.float64), np.swapaxes(np.asarray(k, np.float64), -2, -1))
    if attn_mask is not None:
        s = s * scale + np.asarray(attn_mask, np.float64)
        return np.matmul(softmax_f64(s, 1.0), np.asarray(v, np.float64))
    return np.matmul(softmax_f64(s, scale), np.asarray(v, np.float64))


# ------------------------------------------------------------ brute force

def matmul_bruteforce(a, b) -> list:
    """Triple loop in Python floats (fp64) for tiny 2-D inputs: the
    index-by-index definition C[i][j] = sum_k A[i][k] B[k][j]."""
    m, k = len(a), len(a[0])
    n = len(b[0])
    assert len(b) == k
    return [[math.fsum(float(a[i][p]) * float(b[p][j]) for p in range(k)) for j in range(n)]
            for i in range(m)]
