"""scaffolding_amd — Scaffolding's matmul hot path on MI355X (gfx950).

A drop-in for the reference's GPU matmul path: ``Tensor`` / ``matmul`` /
``matmul_nt``, ``nn.Linear`` / ``F.linear`` (fused bias + SiLU / GELU-tanh),
``F.scaled_dot_product_attention`` (strided-batched QK^T and PV), all on
hand-written HIP kernels behind libsfgemm's C ABI (include/sfgemm.h) and the
Cython seam ``scaffolding_amd._cuda_ops``.

The package computes on the GPU only: tensors on the CPU device can be
created and moved, but the path's operators raise for them, and importing
the package fails if the native extension has not been built
(``python scaffolding_amd/build.py``).
"""
from . import _cuda_ops as _cuops  # noqa: F401  (fails loudly if not built)
from .dtype import bfloat16, dtype, float16, float32
from .device import device
from .tensor import Tensor, from_numpy, matmul, matmul_nt, tensor, zeros, empty
from . import cuda, nn, backends  # noqa: E402

__all__ = [
    "Tensor", "tensor", "from_numpy", "zeros", "empty", "matmul", "matmul_nt",
    "dtype", "float32", "float16", "bfloat16", "device", "cuda", "nn", "backends",
]
__version__ = "0.1.0"
