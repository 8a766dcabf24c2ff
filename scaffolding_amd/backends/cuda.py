"""``backends.cuda.matmul.allow_tf32`` (reference backends/cuda.py:20-35).

Accepted and recorded, never changes the arithmetic: the fp32 GEMM always
runs true fp32 MFMA (gfx950 has no reduced-precision fp32 matrix mode), so
results are identical either way.
"""
from __future__ import annotations

from .. import _cuda_ops as _cuops


class _MatmulFlags:
    def __init__(self):
        self._allow_tf32 = False

    @property
    def allow_tf32(self) -> bool:
        return self._allow_tf32

    @allow_tf32.setter
    def allow_tf32(self, value: bool) -> None:
        self._allow_tf32 = bool(value)
        _cuops.set_tf32_enabled(self._allow_tf32)


matmul = _MatmulFlags()
