"""The reference's DiT block glue, restated in NumPy (test infrastructure;
never imported by the product path).

fp32 restatement of the reference's CPU code, line for line in meaning:

  layer_norm      mean, var (population), (x - mean) / sqrt(var + eps),
                  * weight + bias                     reference nn/layers.py:512-521
  rms_norm        x / sqrt(mean(x^2) + eps) * weight  reference nn/layers.py:576-581
  ada_layer_norm  h = layer_norm(x); p = linear(cond);
                  h * (p[..., :C] + 1) + p[..., C:]   reference diffusion/models.py:478-486
  dit_attn        softmax(q k^T / sqrt(D)) v with the reference's
                  max shift and its + 1e-9 in the denominator
                                                      reference diffusion/models.py:529-536
  dit_block       adaLN -> qkv -> head split -> attn -> merge -> out-proj
                  + residual; [cross-attention]; adaLN -> Linear -> SiLU
                  -> (Dropout, identity at p = 0) -> Linear + residual
                                                      reference diffusion/models.py:538-590

The *_f64 functions are the closed forms in float64; dit_block_mirror
evaluates the block in float64 with the result of every device operation
rounded to the device dtype at the same points as the GPU path (the GPU
keeps 16-bit activations between launches), the accuracy oracle of the
block test.  Parameters are a dict keyed like the reference's state_dict
(norm1.norm.weight, norm1.linear.weight, to_qkv.weight, self_out.weight,
ff.0.weight, ff.3.weight, ...).
"""
from __future__ import annotations

import math

import numpy as np

from . import cpu_path as ref
from .quant import quantize


# ---------------------------------------------------------------- fp32 path

def layer_norm(x, weight=None, bias=None, eps: float = 1e-5):
    """reference nn/layers.py:512-521 (one normalised trailing dim)."""
    mean = np.mean(x, axis=-1, keepdims=True)
    var = np.var(x, axis=-1, keepdims=True)
    x_norm = (x - mean) / np.sqrt(var + eps)
    if weight is not None:
        x_norm = x_norm * weight + bias
    return x_norm.astype(np.float32)


def rms_norm(x, weight, eps: float = 1e-6):
    """reference nn/layers.py:576-581."""
    rms = np.sqrt(np.mean(x ** 2, axis=-1, keepdims=True) + eps)
    return (x / rms * weight).astype(np.float32)


def ada_layer_norm(x, cond, p: dict, prefix: str, eps: float = 1e-5):
    """reference diffusion/models.py:478-486: LayerNorm(dim) with its affine
    parameters, then Linear(cond_dim, 2 dim) of cond as (scale, shift)."""
    h = layer_norm(x, p[prefix + ".norm.weight"], p[prefix + ".norm.bias"], eps)
    params = ref.linear(cond, p[prefix + ".linear.weight"], p[prefix + ".linear.bias"])
    c = h.shape[-1]
    scale = params[..., :c] + 1.0
    shift = params[..., c:]
    return (h * scale + shift).astype(np.float32)


def dit_attn(q, k, v):
    """reference diffusion/models.py:529-536, q (B, H, N, D), k, v (B, H, S, D)."""
    d = q.shape[-1]
    scale = 1.0 / math.sqrt(d)
    scores = np.einsum('bhnd,bhmd->bhnm', q, k) * scale
    scores -= scores.max(axis=-1, keepdims=True)
    exp_s = np.exp(scores)
    attn = exp_s / (exp_s.sum(axis=-1, keepdims=True) + 1e-9)
    return np.einsum('bhnm,bhmd->bhnd', attn, v)


def split_heads(t, heads: int):
    """(B, N, C) -> (B, H, N, D): reference diffusion/models.py:555-557."""
    b, n, c = t.shape
    return t.reshape(b, n, heads, c // heads).transpose(0, 2, 1, 3).copy()


def merge_heads(t):
    """(B, H, N, D) -> (B, N, H D): reference diffusion/models.py:559."""
    b, h, n, d = t.shape
    return t.transpose(0, 2, 1, 3).reshape(b, n, h * d).copy()


def dit_block(x, cond, p: dict, heads: int, context=None, eps: float = 1e-5):
    """reference diffusion/models.py:538-590 on float32 arrays, x (B, N, C),
    cond (B, cond_dim) (B == 1, or cond (B, 1, cond_dim)), context
    (B, S, context_dim) or None."""
    c = x.shape[-1]
    h = ada_layer_norm(x, cond, p, "norm1", eps)
    qkv = ref.linear(h, p["to_qkv.weight"])
    q, k, v = [split_heads(qkv[:, :, i * c:(i + 1) * c], heads) for i in range(3)]
    sa = merge_heads(dit_attn(q, k, v))
    sa_t = ref.linear(sa.astype(np.float32), p["self_out.weight"], p["self_out.bias"])
    x = (x + sa_t).astype(np.float32)
    if context is not None and "cross_q.weight" in p:
        h2 = ada_layer_norm(x, cond, p, "norm2", eps)
        cq = ref.linear(h2, p["cross_q.weight"])
        ck = ref.linear(context, p["cross_k.weight"])
        cv = ref.linear(context, p["cross_v.weight"])
        ca = merge_heads(dit_attn(split_heads(cq, heads), split_heads(ck, heads), split_heads(cv, heads)))
        ca_out = ref.linear(ca.astype(np.float32), p["cross_out.weight"], p["cross_out.bias"])
        x = (x + ca_out).astype(np.float32)
    ff_in = ada_layer_norm(x, cond, p, "norm3", eps)
    f = ref.silu(ref.linear(ff_in, p["ff.0.weight"], p["ff.0.bias"]))
    ff_out = ref.linear(f, p["ff.3.weight"], p["ff.3.bias"])
    return (x + ff_out).astype(np.float32)


# ---------------------------------------------------------------- float64 closed forms

def layer_norm_f64(x, gamma=None, beta=None, eps: float = 1e-5, mod_scale=None, mod_shift=None):
    """float64 (x - mu) / sqrt(var + eps) * gamma + beta, then
    * (1 + mod_scale) + mod_shift (broadcast over the rows of each group)."""
    x = np.asarray(x, np.float64)
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    h = (x - mu) / np.sqrt(var + eps)
    if gamma is not None:
        h = h * np.asarray(gamma, np.float64)
    if beta is not None:
        h = h + np.asarray(beta, np.float64)
    if mod_scale is not None:
        h = h * (1.0 + np.asarray(mod_scale, np.float64))
    if mod_shift is not None:
        h = h + np.asarray(mod_shift, np.float64)
    return h


def rms_norm_f64(x, gamma=None, eps: float = 1e-6):
    x = np.asarray(x, np.float64)
    y = x / np.sqrt((x ** 2).mean(axis=-1, keepdims=True) + eps)
    return y if gamma is None else y * np.asarray(gamma, np.float64)


def mha_f64(q, k, v, heads: int, scale: float | None = None):
    """float64 attention over heads packed in the last dim: q (B, N, C),
    k, v (B, S, C) -> (B, N, C)."""
    d = q.shape[-1] // heads
    s = 1.0 / math.sqrt(d) if scale is None else scale
    o = ref.sdpa_f64(split_heads(np.asarray(q, np.float64), heads), split_heads(np.asarray(k, np.float64), heads),
                     split_heads(np.asarray(v, np.float64), heads), s)
    return merge_heads(o)


def dit_block_mirror(x, cond, p: dict, heads: int, dtype: str | None, context=None, eps: float = 1e-5):
    """The block in float64 with every device operation's output rounded to
    `dtype`, at the GPU path's launch boundaries: the three adaLN
    projections, the three fused adaLN norms, the QKV projection, the fused
    attention, the out-projection with its residual, the SiLU up-projection
    and the down-projection with its residual (plus the cross-attention
    launches when a context is given).  Inputs and parameters must already
    be representable in `dtype`; dtype None rounds nothing (the float64
    closed form of the whole block)."""
    def q(a):
        if dtype is None:  # no rounding: the plain float64 closed form
            return np.asarray(a, np.float64)
        return quantize(np.asarray(a, np.float64).astype(np.float32), dtype).astype(np.float64)

    c = x.shape[-1]

    def ada(xx, prefix):
        params = q(ref.linear_f64(cond, p[prefix + ".linear.weight"], p[prefix + ".linear.bias"]))
        params = params.reshape(params.shape[0], 1, 2 * c)
        return q(layer_norm_f64(xx, p[prefix + ".norm.weight"], p[prefix + ".norm.bias"], eps,
                                params[..., :c], params[..., c:]))

    x = np.asarray(x, np.float64)
    h = ada(x, "norm1")
    qkv = q(ref.linear_f64(h, p["to_qkv.weight"]))
    sa = q(mha_f64(qkv[..., :c], qkv[..., c:2 * c], qkv[..., 2 * c:], heads))
    x = q(ref.linear_f64(sa, p["self_out.weight"], p["self_out.bias"]) + x)
    if context is not None and "cross_q.weight" in p:
        h2 = ada(x, "norm2")
        cq = q(ref.linear_f64(h2, p["cross_q.weight"]))
        ck = q(ref.linear_f64(context, p["cross_k.weight"]))
        cv = q(ref.linear_f64(context, p["cross_v.weight"]))
        ca = q(mha_f64(cq, ck, cv, heads))
        x = q(ref.linear_f64(ca, p["cross_out.weight"], p["cross_out.bias"]) + x)
    ff_in = ada(x, "norm3")
    f = q(ref.linear_f64(ff_in, p["ff.0.weight"], p["ff.0.bias"], "silu"))
    return q(ref.linear_f64(f, p["ff.3.weight"], p["ff.3.bias"]) + x)
