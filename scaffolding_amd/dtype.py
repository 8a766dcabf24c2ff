"""Dtypes of the path (reference dtype.py:1-73).

The reference maps ``bfloat16`` to NumPy float32 (reference dtype.py:31),
i.e. it has no 16-bit brain-float storage.  Here ``bfloat16`` is real 2-byte
device storage (``_cuda_ops.BFLOAT16``); host views of it are float32.
"""
from __future__ import annotations

import enum

import numpy as np

from . import _cuda_ops as _cuops


class dtype(enum.Enum):
    float16 = "float16"
    float32 = "float32"
    bfloat16 = "bfloat16"

    def to_numpy(self) -> np.dtype:
        """Host dtype of this dtype's values (reference dtype.py:25-39)."""
        return np.dtype(np.float16) if self is dtype.float16 else np.dtype(np.float32)

    def device_storage(self) -> np.dtype:
        """Storage dtype of a device tensor of this dtype."""
        if self is dtype.bfloat16:
            return _cuops.BFLOAT16
        return np.dtype(self.value)

    @staticmethod
    def from_any(d) -> "dtype":
        if isinstance(d, dtype):
            return d
        if isinstance(d, str):
            return dtype(d)
        nd = np.dtype(d)
        if nd == _cuops.BFLOAT16:
            return dtype.bfloat16
        if nd == np.float16:
            return dtype.float16
        if nd in (np.float32, np.float64):
            return dtype.float32
        raise TypeError("unsupported dtype %r" % (d,))

    @property
    def itemsize(self) -> int:
        return 4 if self is dtype.float32 else 2

    def __repr__(self) -> str:
        return "scaffolding_amd." + self.value


float16 = dtype.float16
float32 = dtype.float32
bfloat16 = dtype.bfloat16
