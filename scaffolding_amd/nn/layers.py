"""Module, Parameter, Linear, SiLU, GELU (reference nn/module.py,
nn/parameter.py, nn/layers.py:59-151, :358-440).

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
        return {n: p.numpy() for n, p in self.named_parameters()}

    def load_state_dict(self, state: dict) -> None:
        own = dict(self.named_parameters())
        missing = set(own) - set(state)
        if missing:
            raise KeyError("missing keys: %s" % sorted(missing))
        for name, arr in state.items():
            target = own[name]
            owner = self
            parts = name.split(".")
            for part in parts[:-1]:
                owner = owner._modules[part]
            if tuple(np.shape(arr)) != target.shape:
                raise ValueError("shape mismatch for %s: %s vs %s" % (name, np.shape(arr), target.shape))
            setattr(owner, parts[-1], Parameter(Tensor(arr, dtype=target.dtype, device=target.device),
                                                requires_grad=target.requires_grad))


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

    def forward(self, x: Tensor, activation: str | None = None) -> Tensor:
        act = activation if activation is not None else self.activation
        return _linear(x, self.weight, self.bias, act)

    def __repr__(self) -> str:
        return "Linear(in_features=%d, out_features=%d, bias=%s)" % (
            self.in_features, self.out_features, self.bias is not None)


def _linear(x: Tensor, weight: Tensor, bias: Tensor | None, act: str | None) -> Tensor:
    if x._gpu is None or weight._gpu is None or (bias is not None and bias._gpu is None):
        _gpu_only("linear")
    dev = x._gpu.device_id
    w_gt = weight._gpu
    if w_gt.device_id != dev:
        w_gt = _cuops.gputensor_to_device(w_gt, dev)
    b_gt = None
    if bias is not None:
        b_gt = bias._gpu if bias._gpu.device_id == dev else _cuops.gputensor_to_device(bias._gpu, dev)
    _cuops.set_device(dev)
    return Tensor._wrap_gpu(_cuops.dev_linear_forward(x._gpu, w_gt, b_gt, act), x._device)


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


__all__ = ["Module", "Parameter", "Linear", "SiLU", "GELU", "_device_t", "_dtype_t"]
