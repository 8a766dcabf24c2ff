"""Shared helpers of the parity tests: device upload/download and the error
bounds the checks use."""
from __future__ import annotations

import numpy as np

from oracle import cpu_path as ref
from oracle.quant import quantize

STORAGE = {"float32": np.float32, "float16": np.float16}


def cu():
    from scaffolding_amd import _cuda_ops
    return _cuda_ops


def storage(dtype: str):
    if dtype == "bfloat16":
        return cu().BFLOAT16
    return np.dtype(STORAGE[dtype])


def up(x, dtype: str):
    """Uploads float32 values (already representable in `dtype`) as a device
    tensor of `dtype`; 16-bit storage is produced by the device cast."""
    return cu().gputensor_from_numpy(np.ascontiguousarray(x, dtype=np.float32), -1, storage(dtype))


def down(gt) -> np.ndarray:
    return cu().gputensor_to_numpy(gt).astype(np.float32)


def out_half_ulp_rel(dtype: str) -> float:
    """Relative half-ulp of round-to-nearest into the output dtype."""
    return {"float32": 2.0 ** -24, "float16": 2.0 ** -11, "bfloat16": 2.0 ** -8}[dtype]


def gemm_bound(y64: np.ndarray, absprod: np.ndarray, k: int, dtype: str, act: str | None = None):
    """Elementwise bound on |y - y64| for a GEMM with fp32 accumulation over
    k terms (|error| <= k * 2^-23 * sum|a||b|, generous), the fp32 epilogue
    (a few ulps, 1e-6 relative) and one rounding into `dtype` (half ulp of
    the value, plus dtype-subnormal spacing).  Activations used here have
    slope <= 1.13, so the pre-activation error is scaled by 1.2."""
    acc = k * 2.0 ** -23 * absprod
    lip = 1.2 if act else 1.0
    sub = {"float32": 2.0 ** -149, "float16": 2.0 ** -25, "bfloat16": 2.0 ** -133}[dtype]
    return (1.0 + 1e-6) * (lip * acc + (out_half_ulp_rel(dtype) + 2e-6) * np.abs(y64)) + 1e-7 + sub


def check_bound(y, y64, bound, what=""):
    err = np.abs(np.asarray(y, np.float64) - y64)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError("%s: %d of %d elements out of bound; worst at %s: y=%r ref=%r "
                             "err=%.3e bound=%.3e" % (what, int(bad.sum()), err.size, i, float(y[i]),
                                                      float(y64[i]), float(err[i]), float(bound[i])))


def sample_rows(m: int, count: int, seed: int, tile: int = 256) -> np.ndarray:
    """Row indices: both ends, tile edges, the last (possibly ragged) tile,
    and a seeded random sample.

    Every tile edge pair (t - 1, t) is kept while there are at most 32 of
    them; past that, 32 pairs evenly spaced over the tiles, the last tile's
    always among them.  The last tile contributes its first two, middle and
    last two rows, so a ragged tail is checked at any M."""
    last = ((m - 1) // tile) * tile
    keep = {0, 1, m - 2, m - 1, last - 1, last, last + 1, (last + m - 1) // 2}
    starts = list(range(tile, m, tile))
    if len(starts) > 32:
        pick = np.unique(np.linspace(0, len(starts) - 1, 32).round().astype(np.int64))
        starts = [starts[i] for i in pick]
    for t in starts:
        keep.update({t - 1, t})
    edges = np.array(sorted(e for e in keep if 0 <= e < m), dtype=np.int64)
    rng = np.random.default_rng(seed)
    extra = rng.choice(m, size=min(count, m), replace=False)
    return np.unique(np.concatenate([edges, extra]))


def rnd(rng, shape, std, dtype):
    return quantize((rng.standard_normal(shape) * std).astype(np.float32), dtype)


__all__ = ["ref", "quantize", "up", "down", "gemm_bound", "check_bound", "sample_rows", "rnd",
           "storage", "cu"]
