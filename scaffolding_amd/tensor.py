"""Tensor and the matmul entry points of the path.

Mirrors the reference's GPU-resident branch of ``Tensor`` (reference
tensor.py:66-113, :293-320) and ``matmul`` / ``matmul_nt`` (reference
tensor.py:1480-1539): a CUDA-device tensor owns a ``GpuTensor`` (``_gpu``)
and the operators dispatch straight to ``_cuda_ops.dev_*``; results are
wrapped without a grad_fn, as the reference's GPU branch does
(tensor.py:1487-1489).  CPU-device tensors exist for construction and
transfer only: the path computes on the GPU, so operators raise for them.
"""
from __future__ import annotations

import numpy as np

from . import _cuda_ops as _cuops
from .device import device as _device_t
from .dtype import dtype as _dtype_t


def _gpu_only(op: str):
    raise RuntimeError("%s: scaffolding_amd computes the matmul path on the GPU only; "
                       "move the tensors with .to('cuda')" % op)


class Tensor:
    __slots__ = ("_data", "_gpu", "_device", "_dtype", "_requires_grad")

    def __init__(self, data=None, dtype=None, device=None, requires_grad: bool = False):
        self._gpu = None
        self._data = None
        self._device = _device_t(device or "cpu")
        self._requires_grad = bool(requires_grad)
        if data is None:
            self._dtype = _dtype_t.from_any(dtype or "float32")
            return
        arr = np.asarray(data)
        self._dtype = _dtype_t.from_any(dtype if dtype is not None else
                                        (arr.dtype if arr.dtype == np.float16 else "float32"))
        host = arr.astype(self._dtype.to_numpy(), copy=False)
        if self._device.is_cuda:
            self._gpu = _cuops.gputensor_from_numpy(np.ascontiguousarray(host), self._device.ordinal(),
                                                    self._dtype.device_storage())
        else:
            from .dtype import bfloat16
            if self._dtype is bfloat16:
                raise TypeError("bfloat16 tensors live on the GPU only")
            self._data = np.ascontiguousarray(host)

    # -- construction ---------------------------------------------------
    @classmethod
    def _wrap_gpu(cls, gt, device=None, requires_grad: bool = False) -> "Tensor":
        """Wraps a GpuTensor (reference tensor.py:293-305)."""
        t = cls.__new__(cls)
        t._data = None
        t._gpu = gt
        t._device = _device_t(device) if device is not None else _device_t("cuda:%d" % gt.device_id)
        t._dtype = _dtype_t.from_any(gt.dtype)
        t._requires_grad = requires_grad
        return t

    # -- metadata ---------------------------------------------------------
    @property
    def shape(self) -> tuple:
        return tuple(self._gpu.shape) if self._gpu is not None else tuple(self._data.shape)

    @property
    def ndim(self) -> int:
        return len(self.shape)

    @property
    def dtype(self) -> _dtype_t:
        return self._dtype

    @property
    def device(self) -> _device_t:
        return self._device

    @property
    def requires_grad(self) -> bool:
        return self._requires_grad

    @property
    def is_cuda(self) -> bool:
        return self._device.is_cuda

    def numel(self) -> int:
        n = 1
        for s in self.shape:
            n *= s
        return n

    def size(self, dim: int | None = None):
        return self.shape if dim is None else self.shape[dim]

    def __repr__(self) -> str:
        return "Tensor(shape=%s, dtype=%s, device=%s)" % (self.shape, self._dtype.value, self._device)

    # -- transfer ---------------------------------------------------------
    def numpy(self) -> np.ndarray:
        if self._gpu is not None:
            return _cuops.gputensor_to_numpy(self._gpu)
        return self._data

    def to(self, device=None, dtype=None) -> "Tensor":
        dev = _device_t(device) if device is not None else self._device
        dt = _dtype_t.from_any(dtype) if dtype is not None else self._dtype
        if dev.is_cuda:
            if self._gpu is not None:
                gt = self._gpu
                if gt.device_id != dev.ordinal():
                    gt = _cuops.gputensor_to_device(gt, dev.ordinal())
                if dt is not self._dtype:
                    gt = _cuops.dev_cast(gt, dt.device_storage())
                return Tensor._wrap_gpu(gt, dev, self._requires_grad)
            return Tensor(self._data, dtype=dt, device=dev, requires_grad=self._requires_grad)
        host = self.numpy()
        return Tensor(host, dtype=dt, device="cpu", requires_grad=self._requires_grad)

    def cuda(self, index: int = 0) -> "Tensor":
        return self.to("cuda:%d" % index)

    def cpu(self) -> "Tensor":
        return self.to("cpu")

    def reshape(self, *shape) -> "Tensor":
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        shape = list(shape)
        if -1 in shape:
            i = shape.index(-1)
            rest = 1
            for j, s in enumerate(shape):
                if j != i:
                    rest *= s
            shape[i] = self.numel() // rest if rest else 0
        if self._gpu is not None:
            return Tensor._wrap_gpu(_cuops.dev_reshape(self._gpu, tuple(shape)), self._device,
                                    self._requires_grad)
        t = Tensor(self._data.reshape(shape), device="cpu", requires_grad=self._requires_grad)
        return t

    view = reshape

    # -- operators on the path -------------------------------------------
    def matmul(self, other: "Tensor") -> "Tensor":
        return matmul(self, other)

    def __matmul__(self, other: "Tensor") -> "Tensor":
        return matmul(self, other)


def tensor(data, dtype=None, device=None, requires_grad: bool = False) -> Tensor:
    return Tensor(data, dtype=dtype, device=device, requires_grad=requires_grad)


def from_numpy(arr: np.ndarray, device=None, dtype=None) -> Tensor:
    return Tensor(arr, dtype=dtype, device=device)


def zeros(*shape, dtype=None, device="cuda") -> Tensor:
    if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
        shape = tuple(shape[0])
    dt = _dtype_t.from_any(dtype or "float32")
    dev = _device_t(device)
    if not dev.is_cuda:
        return Tensor(np.zeros(shape, dt.to_numpy()), dtype=dt, device=dev)
    return Tensor._wrap_gpu(_cuops.zeros(tuple(shape), dt.device_storage(), dev.ordinal()), dev)


def empty(*shape, dtype=None, device="cuda") -> Tensor:
    if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
        shape = tuple(shape[0])
    dt = _dtype_t.from_any(dtype or "float32")
    dev = _device_t(device)
    if not dev.is_cuda:
        return Tensor(np.empty(shape, dt.to_numpy()), dtype=dt, device=dev)
    return Tensor._wrap_gpu(_cuops.empty(tuple(shape), dt.device_storage(), dev.ordinal()), dev)


def _both_gpu(a: Tensor, b: Tensor, op: str) -> None:
    if a._gpu is None or b._gpu is None:
        _gpu_only(op)
    if a._gpu.device_id != b._gpu.device_id:
        raise RuntimeError("%s: operands on different devices (%s, %s)" % (op, a.device, b.device))


def matmul(a: Tensor, b: Tensor) -> Tensor:
    """reference tensor.py:1480-1489: 2-D -> dev_matmul, any operand >= 3-D
    -> dev_batched_matmul (np.matmul's batch broadcast of a 2-D operand).

    A 1-D operand, which the reference hands to np.matmul on the host
    (tensor.py:1494-1497), stays on the device with np.matmul's rules: a
    vector on the left is a (1, K) row, on the right a (K, 1) column (both
    metadata-only views), and that axis is dropped from the result."""
    _both_gpu(a, b, "matmul")
    if a.ndim == 0 or b.ndim == 0:
        raise ValueError("matmul: operands must be at least 1-D (shapes %s, %s)" % (a.shape, b.shape))
    ga, gb = a._gpu, b._gpu
    if a.ndim == 1:
        ga = _cuops.dev_reshape(ga, (1, a.shape[0]))
    if b.ndim == 1:
        gb = _cuops.dev_reshape(gb, (b.shape[0], 1))
    if len(ga.shape) == 2 and len(gb.shape) == 2:
        out = _cuops.dev_matmul(ga, gb)
    else:
        out = _cuops.dev_batched_matmul(ga, gb)
    if a.ndim == 1 or b.ndim == 1:
        shape = tuple(out.shape)
        if b.ndim == 1:
            shape = shape[:-1]
        if a.ndim == 1:
            shape = shape[:-1] if b.ndim == 1 else shape[:-2] + shape[-1:]
        out = _cuops.dev_reshape(out, shape)
    return Tensor._wrap_gpu(out, a._device)


def matmul_nt(a: Tensor, b: Tensor, alpha: float = 1.0) -> Tensor:
    """C = alpha * A @ B^T (reference tensor.py:1529-1539; alpha is this
    build's fused scale, default 1)."""
    _both_gpu(a, b, "matmul_nt")
    if a.ndim == 2 and b.ndim == 2:
        out = _cuops.dev_matmul_nt(a._gpu, b._gpu, alpha)
    elif a.ndim >= 2 and b.ndim >= 2:
        out = _cuops.dev_batched_matmul_nt(a._gpu, b._gpu, alpha)
    else:
        raise ValueError("matmul_nt: operands must be at least 2-D")
    return Tensor._wrap_gpu(out, a._device)
