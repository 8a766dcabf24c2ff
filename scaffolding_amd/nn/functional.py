"""Functional ops of the path (reference nn/functional.py).

  linear                          reference nn/functional.py:374-395
  silu / gelu (tanh)              reference nn/functional.py:37-89
  softmax                         reference nn/functional.py:113-145
  dropout                         reference nn/functional.py:231-238
  scaled_dot_product_attention    reference nn/functional.py:298-369

GPU only; results carry no grad_fn (as the reference's GPU branches).
"""
from __future__ import annotations

import math

from .. import _cuda_ops as _cuops
from ..tensor import Tensor, _gpu_only
from .layers import _linear


def linear(input: Tensor, weight: Tensor, bias: Tensor | None = None,
           activation: str | None = None) -> Tensor:
    return _linear(input, weight, bias, activation)


def silu(input: Tensor) -> Tensor:
    if input._gpu is None:
        _gpu_only("silu")
    return Tensor._wrap_gpu(_cuops.dev_silu(input._gpu), input._device)


def gelu(input: Tensor, approximate: str = "tanh") -> Tensor:
    if input._gpu is None:
        _gpu_only("gelu")
    if approximate != "tanh":
        raise NotImplementedError("only the tanh approximation is on the device path")
    return Tensor._wrap_gpu(_cuops.dev_gelu(input._gpu), input._device)


def softmax(input: Tensor, dim: int = -1, dtype=None) -> Tensor:
    if input._gpu is None:
        _gpu_only("softmax")
    if dtype is not None:
        raise NotImplementedError("softmax(dtype=...) is not on the device path")
    return Tensor._wrap_gpu(_cuops.dev_softmax(input._gpu, dim), input._device)


def dropout(input: Tensor, p: float = 0.5, training: bool = True) -> Tensor:
    """Zeroes each element with probability p and scales the rest by
    1 / (1 - p) (reference nn/functional.py:231-238, GPU branch
    dev_dropout); identity when not training or p == 0.  Each call draws
    the next stream of the device random state (scaffolding_amd.cuda
    .manual_seed); the reference's GPU branch passes seed 0 every call."""
    if not training or p == 0.0:
        return input
    if input._gpu is None:
        _gpu_only("dropout")
    seed, offset = _cuops.next_random_stream()
    out, _ = _cuops.dev_dropout(input._gpu, p, seed, offset, False)
    return Tensor._wrap_gpu(out, input._device)


def scaled_dot_product_attention(q: Tensor, k: Tensor, v: Tensor, attn_mask=None,
                                 dropout_p: float = 0.0, scale: float | None = None) -> Tensor:
    """softmax(scale * q k^T + attn_mask) v, scale defaulting to 1/sqrt(head
    size).  16-bit inputs with a head size that is a multiple of 8 up to 64
    and no mask run as one fused launch (sf_attention: the scores never
    reach memory); other inputs take three launches: a strided-batched QK^T
    with the scale in its epilogue, a row softmax with the additive mask
    folded in, and a strided-batched PV.  The reference's GPU path
    (nn/functional.py:310-321) runs a Python loop of per-head SGEMMs, a
    scale pass, the softmax and a batched SGEMM, and sends a masked call to
    its host branch (:339-341: scores += mask, NumPy broadcasting); here
    the mask (a Tensor on the device, or a host array or CPU Tensor, which
    is uploaded) is applied on the device with the same broadcasting.
    dropout_p > 0 drops attention weights before PV as the reference's GPU
    branch does (:317-318), on the three-launch path, with the next stream
    of the device random state (see dropout)."""
    if q._gpu is None or k._gpu is None or v._gpu is None:
        _gpu_only("scaled_dot_product_attention")
    seed, offset = _cuops.next_random_stream() if dropout_p > 0.0 else (0, 0)
    mask = None
    if attn_mask is not None:
        if isinstance(attn_mask, Tensor):
            mask = attn_mask._gpu if attn_mask._gpu is not None else attn_mask.numpy()
        else:
            mask = attn_mask
    d = q.shape[-1]
    s = (1.0 / math.sqrt(d)) if scale is None else float(scale)
    out = _cuops.dev_scaled_dot_product_attention(q._gpu, k._gpu, v._gpu, s, mask, dropout_p, seed, offset)
    return Tensor._wrap_gpu(out, q._device)
