"""AdaLayerNorm and DiTBlock on the device (reference
diffusion/models.py:470-590).

The reference evaluates the block on the host: every projection result is
pulled back (``_ensure_cpu``), the adaptive norm's scale / shift, the head
split / merge, the attention and the residual adds run in NumPy.  Here the
block stays in device memory from input to output, in eight launches for
self-attention plus the MLP:

  adaLN-1   skinny Linear(cond) -> (scale, shift); one fused layer norm +
            modulation (sf_layer_norm)
  qkv       one GEMM
  attention one fused kernel reading Q, K, V in place from the packed qkv
            and writing the merged heads (sf_attention_heads)
  out-proj  one GEMM with bias and the residual x fused (sf_gemm_add)
  adaLN-3   as adaLN-1
  MLP       Linear + SiLU fused; Linear + bias + residual fused

State-dict keys equal the reference's (norm1.norm.weight, norm1.linear.*,
to_qkv.weight, self_out.*, [norm2.*, cross_q/k/v.weight, cross_out.*],
norm3.*, ff.0.*, ff.3.*), so its checkpoints load unchanged.  Inference
only, as the reference's GPU branches are (no grad_fn).
"""
from __future__ import annotations

from .. import _cuda_ops as _cuops
from ..nn.layers import Dropout, LayerNorm, Linear, Module, Sequential, SiLU, _on
from ..tensor import Tensor, _gpu_only


class AdaLayerNorm(Module):
    """LayerNorm(dim) followed by h * (1 + scale) + shift, (scale, shift) =
    Linear(cond_dim, 2 dim)(cond) (reference diffusion/models.py:470-486).
    The norm, its affine and the modulation are one launch; the modulation
    row of batch entry b applies to all of its tokens."""

    def __init__(self, dim: int, cond_dim: int, device=None, dtype=None):
        super().__init__()
        self.norm = LayerNorm(dim, device=device, dtype=dtype)
        self.linear = Linear(cond_dim, dim * 2, device=device, dtype=dtype)

    def forward(self, x: Tensor, cond: Tensor) -> Tensor:
        if x._gpu is None or cond._gpu is None:
            _gpu_only("AdaLayerNorm")
        params = self.linear(cond)
        dev = x._gpu.device_id
        _cuops.set_device(dev)
        out = _cuops.dev_ada_layer_norm(x._gpu, _on(params, dev), self.norm.eps, _on(self.norm.weight, dev),
                                        _on(self.norm.bias, dev))
        return Tensor._wrap_gpu(out, x._device)


class DiTBlock(Module):
    """adaLN -> self-attention -> residual, [adaLN -> cross-attention ->
    residual], adaLN -> FFN (Linear, SiLU, Dropout, Linear) -> residual
    (reference diffusion/models.py:490-590).  x (B, N, dim), cond
    (B, cond_dim), context (B, S, context_dim) or None."""

    def __init__(self, dim: int, num_heads: int, cond_dim: int, context_dim: int = 0, dropout: float = 0.0,
                 device=None, dtype=None):
        super().__init__()
        if dim % num_heads != 0:
            raise ValueError("DiTBlock: dim %d is not divisible by num_heads %d" % (dim, num_heads))
        self.dim = dim
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        kw = dict(device=device, dtype=dtype)
        self.norm1 = AdaLayerNorm(dim, cond_dim, **kw)
        self.to_qkv = Linear(dim, dim * 3, bias=False, **kw)
        self.self_out = Linear(dim, dim, **kw)
        self.has_cross = context_dim > 0
        if self.has_cross:
            self.norm2 = AdaLayerNorm(dim, cond_dim, **kw)
            self.cross_q = Linear(dim, dim, bias=False, **kw)
            self.cross_k = Linear(context_dim, dim, bias=False, **kw)
            self.cross_v = Linear(context_dim, dim, bias=False, **kw)
            self.cross_out = Linear(dim, dim, **kw)
        self.norm3 = AdaLayerNorm(dim, cond_dim, **kw)
        self.ff = Sequential(Linear(dim, dim * 4, **kw), SiLU(), Dropout(dropout), Linear(dim * 4, dim, **kw))

    def forward(self, x: Tensor, cond: Tensor, context: Tensor | None = None) -> Tensor:
        if x._gpu is None or cond._gpu is None or (context is not None and context._gpu is None):
            _gpu_only("DiTBlock")
        if len(x.shape) != 3 or x.shape[-1] != self.dim:
            raise ValueError("DiTBlock: x must be (B, N, %d), got %s" % (self.dim, x.shape))
        dev = x._gpu.device_id
        # ---- self-attention: heads read in place from the packed qkv ----
        h = self.norm1(x, cond)
        qkv = self.to_qkv(h)
        _cuops.set_device(dev)
        sa = Tensor._wrap_gpu(_cuops.dev_attention_packed(qkv._gpu, self.num_heads), x._device)
        x = self.self_out(sa, residual=x)
        # ---- cross-attention ----
        if self.has_cross and context is not None:
            h2 = self.norm2(x, cond)
            cq, ck, cv = self.cross_q(h2), self.cross_k(context), self.cross_v(context)
            _cuops.set_device(dev)
            ca = Tensor._wrap_gpu(_cuops.dev_multihead_attention(cq._gpu, ck._gpu, cv._gpu, self.num_heads),
                                  x._device)
            x = self.cross_out(ca, residual=x)
        # ---- FFN: SiLU fused into the up-projection, residual into the down ----
        ff_in = self.norm3(x, cond)
        up, act, drop, down = self.ff[0], self.ff[1], self.ff[2], self.ff[3]
        if not isinstance(act, SiLU):
            raise NotImplementedError("DiTBlock: the fused FFN expects ff[1] to be SiLU")
        f = drop(up(ff_in, activation="silu"))
        return down(f, residual=x)
