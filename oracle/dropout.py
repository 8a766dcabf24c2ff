"""Dropout's mask, restated in NumPy (test infrastructure; never imported by
the product path).

The reference's device dropout (_cuda_kernels.cu:1431-1480, bound at
_cuda_ops.pyx:1243-1255 and called by nn/functional.py:231-238 and, for the
attention weights, :317-318) keeps element i with probability 1 - p and then
scales it by 1 / (1 - p):

    mask[i] = 1 / (1 - p) if u_i >= p else 0,     y[i] = x[i] * mask[i]

with u_i uniform in [0, 1).  The reference draws u from cuRAND's
Philox4x32-10 stream, whose element mapping is part of a closed library and
is not restated here; this library draws u from its own counter-based
Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
easy as 1, 2, 3", SC 2011; the public Random123 algorithm), so the masks
agree with the reference in law (each element kept independently with
probability 1 - p, the same scale), not bit for bit.  This file is the
checker for this library's own stream:

    key     = (seed mod 2^32, seed >> 32)
    counter = (g mod 2^32, g >> 32, offset mod 2^32, offset >> 32), g = i // 4
    r       = philox4x32_10(counter, key)[i mod 4]
    u_i     = (r >> 8) * 2^-24

philox4x32_10 is pinned by the published Random123 known-answer vectors
(tests/test_oracle_dropout.py).
"""
from __future__ import annotations

import numpy as np

M0 = np.uint64(0xD2511F53)
M1 = np.uint64(0xCD9E8D57)
W0 = np.uint32(0x9E3779B9)
W1 = np.uint32(0xBB67AE85)
_MASK32 = np.uint64(0xFFFFFFFF)


def philox4x32_10(ctr: np.ndarray, key: np.ndarray) -> np.ndarray:
    """Philox4x32 with 10 rounds over arrays of counters.

    ctr: uint32 [..., 4]; key: uint32 [..., 2] (broadcast against ctr).
    Each round: (hi0, lo0) = M0 * c0, (hi1, lo1) = M1 * c2 (64-bit
    products), c = (hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0); the key is
    bumped by the Weyl constants (W0, W1) before every round but the
    first."""
    c = np.array(ctr, dtype=np.uint32, copy=True)
    k = np.broadcast_to(np.asarray(key, dtype=np.uint32), c.shape[:-1] + (2,)).copy()
    for r in range(10):
        if r:
            k[..., 0] += W0
            k[..., 1] += W1
        p0 = c[..., 0].astype(np.uint64) * M0
        p1 = c[..., 2].astype(np.uint64) * M1
        hi0 = (p0 >> np.uint64(32)).astype(np.uint32)
        lo0 = (p0 & _MASK32).astype(np.uint32)
        hi1 = (p1 >> np.uint64(32)).astype(np.uint32)
        lo1 = (p1 & _MASK32).astype(np.uint32)
        c = np.stack([hi1 ^ c[..., 1] ^ k[..., 0], lo1, hi0 ^ c[..., 3] ^ k[..., 1], lo0], axis=-1)
    return c


def uniforms(n: int, seed: int, offset: int = 0) -> np.ndarray:
    """u_0 .. u_{n-1} of the stream (seed, offset), float64 in [0, 1)."""
    groups = (n + 3) // 4
    g = np.arange(groups, dtype=np.uint64)
    ctr = np.stack([(g & _MASK32).astype(np.uint32), (g >> np.uint64(32)).astype(np.uint32),
                    np.full(groups, offset & 0xFFFFFFFF, np.uint32),
                    np.full(groups, (offset >> 32) & 0xFFFFFFFF, np.uint32)], axis=-1)
    key = np.array([seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF], np.uint32)
    r = philox4x32_10(ctr, key).reshape(-1)[:n]
    return (r >> np.uint32(8)).astype(np.float64) * 2.0 ** -24


def keep(n: int, p: float, seed: int, offset: int = 0) -> np.ndarray:
    """Boolean keep mask: u_i >= p, with u_i and p compared as float32 (the
    kernel's comparison)."""
    u = uniforms(n, seed, offset).astype(np.float32)
    return u >= np.float32(p)


def dropout(x: np.ndarray, p: float, seed: int, offset: int = 0):
    """(y, mask) in float32: mask = keep * float32(1 / (1 - p)), y = x * mask
    (float32 product; the caller rounds to the storage dtype)."""
    x32 = np.asarray(x, np.float32).reshape(-1)
    scale = np.float32(1.0) / (np.float32(1.0) - np.float32(p))
    m = np.where(keep(x32.size, p, seed, offset), scale, np.float32(0.0)).astype(np.float32)
    return (x32 * m).reshape(np.shape(x)), m.reshape(np.shape(x))
