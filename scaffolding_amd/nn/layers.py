"""Module, Parameter, Sequential, Linear, LayerNorm, RMSNorm, Dropout, SiLU,
GELU (reference nn/module.py, nn/parameter.py, nn/layers.py:59-151,
:339-440, :443-585).

Only the GPU-resident forward of the reference's Linear exists here
(reference nn/layers.py:85-110): weights are uploaded once, on construction
or ``.to()``, and ``forward`` is one ``dev_linear_forward`` launch with the
bias (and, through ``activation``, SiLU / GELU-tanh) fused into the GEMM
epilogue.  The forward is inference-only, as the reference's GPU branch is
(no grad_fn, reference nn/layers.py:108-110).
"""
from __future__ import annotations

import math

import numpy as np

from .. import _cuda_ops as _cuops
from ..device import device as _device_t
from ..dtype import dtype as _dtype_t
from ..tensor import Tensor, _gpu_only


class Parameter(Tensor):
    """A Tensor registered as a module parameter (reference nn/parameter.py)."""
    __slots__ = ()

    def __init__(self, data=None, requires_grad: bool = True, dtype=None, device=None):
        if isinstance(data, Tensor):
            t = data
            self._data, self._gpu, self._device = t._data, t._gpu, t._device
            self._dtype, self._requires_grad = t._dtype, requires_grad
        else:
            super().__init__(data, dtype=dtype, device=device, requires_grad=requires_grad)


class Module:
    """Minimal module container (reference nn/module.py:1-367)."""

    def __init__(self):
        object.__setattr__(self, "_params", {})
        object.__setattr__(self, "_modules", {})
        object.__setattr__(self, "training", True)

    def __setattr__(self, name, value):
        if isinstance(value, Parameter):
            self._params[name] = value
        elif isinstance(value, Module):
            self._modules[name] = value
        elif name in self.__dict__.get("_params", {}) and value is None:
            self._params.pop(name)
        object.__setattr__(self, name, value)

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)

    def forward(self, *args, **kwargs):
        raise NotImplementedError

    def parameters(self):
        for p in self._params.values():
            yield p
        for m in self._modules.values():
            yield from m.parameters()

    def named_parameters(self, prefix: str = ""):
        for n, p in self._params.items():
            yield prefix + n, p
        for mn, m in self._modules.items():
            yield from m.named_parameters(prefix + mn + ".")

    def to(self, device=None, dtype=None) -> "Module":
        for name, p in list(self._params.items()):
            moved = Parameter(p.to(device, dtype), requires_grad=p.requires_grad)
            setattr(self, name, moved)
        for m in self._modules.values():
            m.to(device, dtype)
        return self

    def cuda(self, index: int = 0) -> "Module":
        return self.to("cuda:%d" % index)

    def eval(self) -> "Module":
        object.__setattr__(self, "training", False)
        return self

    def train(self, mode: bool = True) -> "Module":
        object.__setattr__(self, "training", mode)
        return self

    def state_dict(self) -> dict:
        """Parameter name -> the Parameter itself, in registration order
        (reference nn/module.py:136-154: the dict holds the parameters, not
        copies; .numpy() of a value downloads it)."""
        return dict(self.named_parameters())

    def load_state_dict(self, state_dict: dict, strict: bool = True) -> None:
        """reference nn/module.py:156-185: each key naming one of this
        module's parameters replaces that parameter's data in place (the
        Parameter object is kept); keys naming nothing are ignored and
        parameters the dict does not name keep their data (the reference
        takes `strict` and never raises).  Values are NumPy arrays or
        Tensors.  A parameter on the GPU receives them without a host copy
        being kept: host arrays are uploaded as float32 and rounded to the
        parameter's dtype on the device (bfloat16 / float16 by RNE, sf_cast);
        device tensors are copied (and cast) device-side.  Unlike the
        reference, a value whose shape differs from the parameter's raises
        ValueError instead of being uploaded as is."""
        own = dict(self.named_parameters())
        for name, val in state_dict.items():
            target = own.get(name)
            if target is None:
                continue
            shape = tuple(val.shape) if isinstance(val, Tensor) else tuple(np.shape(val))
            if shape != target.shape:
                raise ValueError("load_state_dict: shape mismatch for %s: %s vs %s" % (name, shape, target.shape))
            if target._gpu is None:
                host = val.numpy() if isinstance(val, Tensor) else np.asarray(val)
                target._data = np.array(host, dtype=target._dtype.to_numpy(), copy=True)
                continue
            dev = target._gpu.device_id
            storage = target._dtype.device_storage()
            if isinstance(val, Tensor) and val._gpu is not None:
                src = val._gpu if val._gpu.device_id == dev else _cuops.gputensor_to_device(val._gpu, dev)
                if _cuops.resolve_dtype(src.dtype) == _cuops.resolve_dtype(storage):
                    dst = _cuops.empty(tuple(src.shape), storage, dev)
                    _cuops.dev_copy(src, dst)
                else:
                    dst = _cuops.dev_cast(src, storage)
            else:
                host = val.numpy() if isinstance(val, Tensor) else np.asarray(val)
                dst = _cuops.gputensor_from_numpy(np.ascontiguousarray(host, dtype=np.float32), dev, storage)
            target._gpu = dst
            target._data = None


class Linear(Module):
    """y = x W^T + b (reference nn/layers.py:59-151).

    W is [out_features, in_features], initialised U(-1/sqrt(in), 1/sqrt(in))
    like the reference (nn/layers.py:68-76), bias likewise.  ``activation``
    ('silu' | 'gelu' | None) selects a fused epilogue; the reference applies
    SiLU / GELU as separate passes."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True, device=None,
                 dtype=None, activation: str | None = None):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.activation = activation
        k = 1.0 / math.sqrt(in_features)
        dev = device or "cuda"
        w = np.random.uniform(-k, k, (out_features, in_features)).astype(np.float32)
        self.weight = Parameter(w, dtype=dtype, device=dev)
        if bias:
            b = np.random.uniform(-k, k, (out_features,)).astype(np.float32)
            self.bias = Parameter(b, dtype=dtype, device=dev)
        else:
            self.bias = None

    def forward(self, x: Tensor, activation: str | None = None, residual: Tensor | None = None) -> Tensor:
        """``residual`` (shape of the output) is added in the same launch,
        after the activation: y = act(x W^T + b) + residual."""
        act = activation if activation is not None else self.activation
        return _linear(x, self.weight, self.bias, act, residual)

    def __repr__(self) -> str:
        return "Linear(in_features=%d, out_features=%d, bias=%s)" % (
            self.in_features, self.out_features, self.bias is not None)


def _on(t: Tensor | None, dev: int):
    """t's GpuTensor on device `dev` (copied there if it lives elsewhere)."""
    if t is None:
        return None
    return t._gpu if t._gpu.device_id == dev else _cuops.gputensor_to_device(t._gpu, dev)


def _linear(x: Tensor, weight: Tensor, bias: Tensor | None, act: str | None,
            residual: Tensor | None = None) -> Tensor:
    if x._gpu is None or weight._gpu is None or (bias is not None and bias._gpu is None) or \
            (residual is not None and residual._gpu is None):
        _gpu_only("linear")
    dev = x._gpu.device_id
    _cuops.set_device(dev)
    out = _cuops.dev_linear_forward(x._gpu, _on(weight, dev), _on(bias, dev), act, _on(residual, dev))
    return Tensor._wrap_gpu(out, x._device)


class Sequential(Module):
    """Children run in order, registered as "0", "1", ... so state_dict keys
    match the reference's (reference nn/module.py:345-367)."""

    def __init__(self, *modules):
        super().__init__()
        object.__setattr__(self, "_seq", list(modules))
        for i, m in enumerate(modules):
            self._modules[str(i)] = m

    def forward(self, x):
        for m in self._seq:
            x = m(x)
        return x

    def __len__(self) -> int:
        return len(self._seq)

    def __getitem__(self, idx):
        return self._seq[idx]

    def __iter__(self):
        return iter(self._seq)


class Dropout(Module):
    """Identity in eval mode or at p = 0; in training, F.dropout (reference
    nn/layers.py:339-353)."""

    def __init__(self, p: float = 0.5):
        super().__init__()
        self.p = p

    def forward(self, x: Tensor) -> Tensor:
        if not self.training or self.p == 0.0:
            return x
        from . import functional as F
        return F.dropout(x, self.p, True)


class LayerNorm(Module):
    """Layer normalisation over the last dim (reference nn/layers.py:443-521):
    weight ones and bias zeros of shape (dim,), eps 1e-5; one launch of
    sf_layer_norm, result in the input dtype."""

    def __init__(self, normalized_shape, eps: float = 1e-5, elementwise_affine: bool = True, device=None,
                 dtype=None):
        super().__init__()
        if isinstance(normalized_shape, int):
            normalized_shape = (normalized_shape,)
        if len(normalized_shape) != 1:
            raise NotImplementedError("LayerNorm over more than the last dim is not on the device path")
        self.normalized_shape = tuple(normalized_shape)
        self.eps = eps
        self.elementwise_affine = elementwise_affine
        dev = device or "cuda"
        if elementwise_affine:
            self.weight = Parameter(np.ones(self.normalized_shape, np.float32), dtype=dtype, device=dev)
            self.bias = Parameter(np.zeros(self.normalized_shape, np.float32), dtype=dtype, device=dev)
        else:
            self.weight = None
            self.bias = None

    def forward(self, x: Tensor) -> Tensor:
        if x._gpu is None:
            _gpu_only("layer_norm")
        dev = x._gpu.device_id
        _cuops.set_device(dev)
        w = _on(self.weight, dev) if self.weight is not None else None
        b = _on(self.bias, dev) if self.bias is not None else None
        return Tensor._wrap_gpu(_cuops.dev_layer_norm(x._gpu, w, b, self.eps), x._device)


class RMSNorm(Module):
    """RMS normalisation over the last dim (reference nn/layers.py:529-585):
    weight ones of shape (dim,), eps 1e-6."""

    def __init__(self, normalized_shape, eps: float = 1e-6, device=None, dtype=None):
        super().__init__()
        if isinstance(normalized_shape, int):
            normalized_shape = (normalized_shape,)
        if len(normalized_shape) != 1:
            raise NotImplementedError("RMSNorm over more than the last dim is not on the device path")
        self.normalized_shape = tuple(normalized_shape)
        self.eps = eps
        self.weight = Parameter(np.ones(self.normalized_shape, np.float32), dtype=dtype, device=device or "cuda")

    def forward(self, x: Tensor) -> Tensor:
        if x._gpu is None:
            _gpu_only("rms_norm")
        dev = x._gpu.device_id
        _cuops.set_device(dev)
        return Tensor._wrap_gpu(_cuops.dev_rms_norm(x._gpu, _on(self.weight, dev), self.eps), x._device)


class SiLU(Module):
    """reference nn/layers.py:358-388."""

    def forward(self, x: Tensor) -> Tensor:
        from .functional import silu
        return silu(x)


class GELU(Module):
    """reference nn/layers.py:415-440 (tanh approximation)."""

    def __init__(self, approximate: str = "tanh"):
        super().__init__()
        if approximate != "tanh":
            raise NotImplementedError("only the tanh approximation is on the device path")

    def forward(self, x: Tensor) -> Tensor:
        from .functional import gelu
        return gelu(x)


__all__ = ["Module", "Parameter", "Sequential", "Linear", "LayerNorm", "RMSNorm", "Dropout", "SiLU", "GELU",
           "_device_t", "_dtype_t"]
