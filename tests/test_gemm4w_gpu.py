"""The one-wave-per-SIMD 256x256 NT kernel (gemm16nt_4w.hpp) against the
8-wave kernel: the planner takes it for one workgroup per tile, no split
parts, K >= 4096 and C rows of a multiple of 64 elements, so the same
product written with a C row stride that is not such a multiple runs the
8-wave kernel.  Both accumulate every output in the same order, so the
results must agree bit for bit; a few sampled rows are also checked
against the fp64 oracle."""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from helpers import check_bound, cu, gemm_bound, ref, rnd, sample_rows, up

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SF_DT = {"bfloat16": 2, "float16": 1}
EPI = {(False, None): 0, (True, None): 1, (True, "silu"): 2, (True, "gelu"): 3, (False, "silu"): 4, (False, "gelu"): 5}


def _lib():
    return ctypes.CDLL(os.path.join(ROOT, "scaffolding_amd", "libsfgemm.so"))


def _f32(bits, dtype):
    """16-bit result bits as float32 values."""
    if dtype == "bfloat16":
        return (bits.astype(np.uint32) << 16).view(np.float32)
    return bits.view(np.float16).astype(np.float32)


def _run(so, m, n, k, dtype, gx, gw, gb, epi, ldc, res=None, ldr=0, in_place=False):
    """x . w^T through sf_gemm (or sf_gemm_add with a residual) into a fresh C
    of row stride ldc; returns the plan name and the raw 16-bit results."""
    I64, P = ctypes.c_int64, ctypes.c_void_p
    plan = cu().gemm_plan(1, m, n, k, 1, gx.data_ptr, k, 0, gw.data_ptr, k, 0, ldc, 0, gx.dtype, epi=epi,
                          ptr_bias=gb.data_ptr if gb is not None else 0)
    out = cu().empty((m, ldc), cu().BFLOAT16 if dtype == "bfloat16" else np.float16, 0)
    bias = P(gb.data_ptr) if gb is not None else None
    dt = SF_DT[dtype]
    if res is None:
        rc = so.sf_gemm(0, 1, I64(m), I64(n), I64(k), I64(1), P(gx.data_ptr), I64(k), I64(0), P(gw.data_ptr),
                        I64(k), I64(0), P(out.data_ptr), I64(ldc), I64(0), dt, dt, ctypes.c_float(1.0), bias, epi,
                        None)
    else:
        if in_place:  # R == C: C starts as the residual
            cu().dev_copy(res, out)
            rp, rld = out.data_ptr, ldc
        else:
            rp, rld = res.data_ptr, ldr
        rc = so.sf_gemm_add(0, 1, I64(m), I64(n), I64(k), I64(1), P(gx.data_ptr), I64(k), I64(0),
                            P(gw.data_ptr), I64(k), I64(0), P(out.data_ptr), I64(ldc), I64(0), dt, dt,
                            ctypes.c_float(1.0), bias, epi, P(rp), I64(rld), I64(0), None)
    assert rc == 0, rc
    cu().device_synchronize()
    return plan, cu().gputensor_bits_to_numpy(out)[:, :n].copy(), out


CASES = [
    # (M, N, K, dtype, bias, act, ldc of the 4-wave run, ldc of the 8-wave run);
    # at least one 256 x 256 tile per CU, one workgroup per tile
    (4096, 4096, 4096, "bfloat16", True, None, 4096, 4104),     # the headline shape
    (4000, 4096, 4096, "bfloat16", True, "silu", 4096, 4104),   # partial last row of tiles
    (4000, 4000, 4096, "bfloat16", True, "gelu", 4032, 4040),   # partial rows and columns
    (4000, 3999, 4096, "float16", True, "silu", 4032, 4040),    # odd N: bias loaded in the epilogue
    (4096, 4096, 8192, "float16", False, None, 4096, 4104),     # K = 8192, no bias
    (4096, 6400, 4096, "bfloat16", False, "gelu", 6400, 6408),  # 400 tiles (a second round), no bias
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "%dx%dx%d-%s-%s%s" % (c[0], c[1], c[2], c[3][0:2],
                                                                            "b" if c[4] else "", c[5] or ""))
def test_wave4_bitwise_equals_8wave(case):
    m, n, k, dtype, has_bias, act, ldc4, ldc8 = case
    rng = np.random.default_rng(m + 3 * n + 7 * k)
    x = rnd(rng, (m, k), 1.0, dtype)
    w = rnd(rng, (n, k), 1.0 / np.sqrt(k), dtype)
    gx, gw = up(x, dtype), up(w, dtype)
    b = rnd(rng, (n,), 0.5, dtype) if has_bias else None
    gb = up(b, dtype) if has_bias else None
    epi = EPI[(has_bias, act)]
    so = _lib()
    plan4, y4, _ = _run(so, m, n, k, dtype, gx, gw, gb, epi, ldc4)
    plan8, y8, _ = _run(so, m, n, k, dtype, gx, gw, gb, epi, ldc8)
    assert plan4.endswith("4-wave"), plan4
    assert plan8.startswith("gemm nt 256x256 lds-dma") and "4-wave" not in plan8, plan8
    mism = np.count_nonzero(y4 != y8)
    assert mism == 0, "%d of %d outputs differ between the kernels" % (mism, y4.size)
    rows = sample_rows(m, 12, seed=m + n)
    y = _f32(y4[rows], dtype)
    y64 = ref.linear_f64(x[rows], w, b, act)
    absprod = np.abs(x[rows].astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    check_bound(y, y64, gemm_bound(y64, absprod, k, dtype, act), "4-wave %s" % (case,))


@pytest.mark.parametrize("in_place", [False, True], ids=["R", "R=C"])
def test_wave4_residual_bitwise_equals_8wave(in_place):
    """sf_gemm_add's residual (a separate R, and R == C) through both kernels."""
    m, n, k, dtype = 4000, 4096, 4096, "bfloat16"
    rng = np.random.default_rng(77 + in_place)
    x = rnd(rng, (m, k), 1.0, dtype)
    w = rnd(rng, (n, k), 1.0 / np.sqrt(k), dtype)
    b = rnd(rng, (n,), 0.5, dtype)
    r = rnd(rng, (m, n), 1.0, dtype)
    gx, gw, gb = up(x, dtype), up(w, dtype), up(b, dtype)
    so = _lib()
    outs = []
    for ldc in (4096, 4104):
        rr = np.zeros((m, ldc), np.float32)
        rr[:, :n] = r
        gr = up(rr, dtype)
        plan, y, _ = _run(so, m, n, k, dtype, gx, gw, gb, 2, ldc, res=gr, ldr=ldc, in_place=in_place)
        assert ("4-wave" in plan) == (ldc == 4096), plan
        outs.append(y)
    mism = np.count_nonzero(outs[0] != outs[1])
    assert mism == 0, "%d outputs differ" % mism
    rows = sample_rows(m, 8, seed=5)
    y = _f32(outs[0][rows], dtype)
    y64 = ref.linear_f64(x[rows], w, b, "silu") + r[rows].astype(np.float64)
    absprod = np.abs(x[rows].astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    check_bound(y, y64, gemm_bound(y64 - r[rows], absprod, k, dtype, "silu") + np.abs(y64) * 2.0 ** -8,
                "4-wave residual")
