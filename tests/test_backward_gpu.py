"""Backward-pass GEMMs and reductions on the GPU: A^T B ("TN", the weight
gradient), all four transpose cases of sf_gemm (the cases of the
reference's cuda_sgemm, _cuda_kernels.cu:1184-1217), the sum over one axis
(bias gradient, reference dev_sum_dim _cuda_ops.pyx:1710-1741) and the
fused linear backward (reference autograd.py:793-822) against the fp64
closed form and the reference's fp32 CPU restatement."""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from helpers import check_bound, cu, down, gemm_bound, out_half_ulp_rel, ref, rnd, up
from oracle.configs import normwise_err, tol_fp32

pytestmark = pytest.mark.gpu

DTYPES = ["float32", "float16", "bfloat16"]
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SHAPES = [(1, 1, 1), (3, 5, 7), (2, 3, 8), (17, 33, 65), (64, 64, 64), (100, 130, 72),
          (129, 257, 200), (16, 48, 4096), (255, 257, 128), (300, 64, 520), (512, 512, 2048)]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_matmul_tn(dtype, shape):
    m, n, k = shape
    rng = np.random.default_rng(3000 + m * 7 + n * 13 + k)
    a = rnd(rng, (k, m), 1.0, dtype)  # stored K x M
    b = rnd(rng, (k, n), 1.0 / np.sqrt(max(k, 1)), dtype)
    y = down(cu().dev_matmul_tn(up(a, dtype), up(b, dtype)))
    assert y.shape == (m, n)
    y64 = ref.matmul_f64(a.T, b)
    absprod = np.abs(a.T.astype(np.float64)) @ np.abs(b.astype(np.float64))
    check_bound(y, y64, gemm_bound(y64, absprod, k, dtype), "tn %s %s" % (dtype, shape))
    if dtype == "float32":
        assert normwise_err(y, ref.matmul_tn(a, b)) <= tol_fp32(k)


def _lib():
    lib = ctypes.CDLL(os.path.join(ROOT, "scaffolding_amd", "libsfgemm.so"))
    lib.sf_last_error.restype = ctypes.c_char_p
    return lib


SFD = {"float32": 0, "float16": 1, "bfloat16": 2}


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)], ids=["NN", "NT", "TN", "TT"])
@pytest.mark.parametrize("shape", [(5, 9, 16), (70, 200, 136), (256, 320, 512), (33, 17, 40)],
                         ids=lambda s: "x".join(map(str, s)))
def test_sf_gemm_four_transposes(dtype, ta, tb, shape):
    """sf_gemm through the C ABI with op(A) = A or A^T and op(B) = B or B^T,
    alpha and a bias epilogue, against the fp64 closed form."""
    m, n, k = shape
    rng = np.random.default_rng(4000 + 10 * ta + tb + m + n + k)
    a = rnd(rng, (k, m) if ta else (m, k), 1.0, dtype)
    b = rnd(rng, (n, k) if tb else (k, n), 1.0 / np.sqrt(k), dtype)
    bias = rnd(rng, (n,), 0.5, dtype)
    ga, gb, gbias = up(a, dtype), up(b, dtype), up(bias, dtype)
    gc = cu().empty((m, n), ga.dtype, 0)
    I64 = ctypes.c_int64
    lib = _lib()
    lda = m if ta else k
    ldb = k if tb else n
    rc = lib.sf_gemm(ta, tb, I64(m), I64(n), I64(k), I64(1), ctypes.c_void_p(ga.data_ptr), I64(lda), I64(0),
                     ctypes.c_void_p(gb.data_ptr), I64(ldb), I64(0), ctypes.c_void_p(gc.data_ptr), I64(n),
                     I64(m * n), SFD[dtype], SFD[dtype], ctypes.c_float(0.5), ctypes.c_void_p(gbias.data_ptr), 1,
                     None)
    assert rc == 0, lib.sf_last_error()
    cu().device_synchronize()
    y = down(gc)
    am = (a.T if ta else a).astype(np.float64)
    bm = (b.T if tb else b).astype(np.float64)
    y64 = 0.5 * (am @ bm) + bias.astype(np.float64)
    absprod = 0.5 * (np.abs(am) @ np.abs(bm)) + np.abs(bias.astype(np.float64))
    check_bound(y, y64, gemm_bound(y64, absprod, k, dtype), "%s ta=%d tb=%d %s" % (dtype, ta, tb, shape))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("bcast", ["none", "b2d", "a2d"])
def test_batched_matmul_tn(dtype, bcast):
    rng = np.random.default_rng(21)
    bshape, m, n, k = (2, 3), 40, 72, 48
    a = rnd(rng, (k, m) if bcast == "a2d" else bshape + (k, m), 1.0, dtype)
    b = rnd(rng, (k, n) if bcast == "b2d" else bshape + (k, n), 1.0 / np.sqrt(k), dtype)
    y = down(cu().dev_batched_matmul_tn(up(a, dtype), up(b, dtype)))
    assert y.shape == bshape + (m, n)
    at = np.swapaxes(a, -2, -1).astype(np.float64)
    y64 = np.matmul(at, b.astype(np.float64))
    absprod = np.matmul(np.abs(at), np.abs(b.astype(np.float64)))
    check_bound(y, y64, gemm_bound(y64, absprod, k, dtype), "batched tn %s %s" % (dtype, bcast))


def _sum_bound(x64, axis, dtype, keepdim=False):
    """fp32 accumulation over n terms plus one rounding into dtype."""
    n = x64.shape[axis]
    s = np.abs(x64).sum(axis=axis, keepdims=keepdim)
    y = x64.sum(axis=axis, keepdims=keepdim)
    return y, n * 2.0 ** -23 * s + out_half_ulp_rel(dtype) * np.abs(y) + 1e-30


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape,dim", [((7,), 0), ((5, 3), 0), ((5, 3), 1), ((4, 6, 5), 1), ((2, 3, 1024), -1),
                                       ((3000, 1920), 0), ((17776, 24), 0), ((300, 1001), 0), ((9, 4100), -1),
                                       ((6, 0, 40), 1)],
                         ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else str(v))
def test_sum_dim(dtype, shape, dim):
    rng = np.random.default_rng(5000 + sum(shape))
    x = rnd(rng, shape, 1.0, dtype)
    gx = up(x, dtype)
    y = down(cu().dev_sum_dim(gx, dim))
    y64, bound = _sum_bound(x.astype(np.float64), dim, dtype)
    want_shape = ref.sum_dim(x, dim).shape or (1,)
    assert y.shape == want_shape
    check_bound(y.reshape(y64.shape), y64, bound, "sum_dim %s %s %d" % (dtype, shape, dim))
    yk = down(cu().dev_sum_dim(gx, dim, True))
    assert yk.shape == ref.sum_dim(x, dim, keepdim=True).shape


def test_sum_dim_is_deterministic():
    """The many-row column sum goes through per-part partials summed in a
    fixed order: two runs give the same bits."""
    rng = np.random.default_rng(77)
    x = up(rnd(rng, (20000, 1920), 1.0, "bfloat16"), "bfloat16")
    a = cu().gputensor_bits_to_numpy(cu().dev_sum_dim(x, 0))
    b = cu().gputensor_bits_to_numpy(cu().dev_sum_dim(x, 0))
    assert np.array_equal(a, b)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("has_bias", [True, False])
@pytest.mark.parametrize("lead,n,k", [((3,), 5, 7), ((2, 9), 6, 16), ((300,), 520, 264), ((4, 128), 384, 192),
                                      ((1,), 1920, 1920)], ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else str(v))
def test_linear_backward(dtype, has_bias, lead, n, k):
    rng = np.random.default_rng(6000 + n + k + len(lead))
    g = rnd(rng, lead + (n,), 1.0, dtype)
    x = rnd(rng, lead + (k,), 1.0, dtype)
    w = rnd(rng, (n, k), 1.0 / np.sqrt(k), dtype)
    gi, gw, gb = cu().dev_linear_backward(up(g, dtype), up(x, dtype), up(w, dtype), has_bias)
    dx64, dw64, db64 = ref.linear_backward_f64(g, x, w)
    m = int(np.prod(lead))
    g2 = np.abs(g.reshape(m, n).astype(np.float64))
    x2 = np.abs(x.reshape(m, k).astype(np.float64))
    dx = down(gi)
    assert dx.shape == x.shape
    check_bound(dx, dx64, gemm_bound(dx64, (g2 @ np.abs(w.astype(np.float64))).reshape(dx64.shape), n, dtype),
                "grad_input %s" % dtype)
    dw = down(gw)
    assert dw.shape == w.shape
    check_bound(dw, dw64, gemm_bound(dw64, g2.T @ x2, m, dtype), "grad_weight %s" % dtype)
    if has_bias:
        db = down(gb)
        assert db.shape == (n,)
        _, bound = _sum_bound(g.reshape(m, n).astype(np.float64), 0, dtype)
        check_bound(db, db64, bound, "grad_bias %s" % dtype)
    else:
        assert gb is None
    if dtype == "float32":
        cpu = ref.linear_backward(g, x, w, has_bias)
        assert normwise_err(dx, cpu[0]) <= tol_fp32(n)
        assert normwise_err(dw, cpu[1]) <= tol_fp32(m)


def test_linear_backward_training_shape():
    """C5's out-projection gradients at 4096 tokens (bf16): dX NN, dW TN over
    4096 rows, db a 4096-row column sum; sampled against fp64."""
    rng = np.random.default_rng(8)
    m, n, k = 4096, 1920, 1920
    g = rnd(rng, (m, n), 1.0, "bfloat16")
    x = rnd(rng, (m, k), 1.0, "bfloat16")
    w = rnd(rng, (n, k), 0.02, "bfloat16")
    gi, gw, gb = cu().dev_linear_backward(up(g, "bfloat16"), up(x, "bfloat16"), up(w, "bfloat16"), True)
    rows = np.array([0, 1, 255, 256, 1000, 1919])
    g64, x64, w64 = g.astype(np.float64), x.astype(np.float64), w.astype(np.float64)
    dx = down(gi)[rows]
    dx64 = g64[rows] @ w64
    check_bound(dx, dx64, gemm_bound(dx64, np.abs(g64[rows]) @ np.abs(w64), n, "bfloat16"), "dX")
    dw = down(gw)[rows]
    dw64 = g64[:, rows].T @ x64
    check_bound(dw, dw64, gemm_bound(dw64, np.abs(g64[:, rows]).T @ np.abs(x64), m, "bfloat16"), "dW")
    db64, bound = _sum_bound(g64, 0, "bfloat16")
    check_bound(down(gb), db64, bound, "db")


LDS_DMA_CASES = [
    # (dtype, transA, transB, M, N, K, batch, epilogue, expected plan)
    ("bfloat16", 0, 0, 4096, 4096, 256, 1, 0, "gemm nn 256x256 lds-dma"),
    ("float16", 1, 0, 4000, 4104, 384, 1, 0, "gemm tn 256x256 lds-dma"),
    ("bfloat16", 1, 1, 4096, 4096, 128, 1, 0, "gemm tt 256x256 lds-dma"),
    ("float16", 0, 0, 1000, 1104, 128, 16, 0, "gemm nn 256x256 lds-dma"),
    ("bfloat16", 1, 0, 1000, 1104, 256, 16, 0, "gemm tn 256x256 lds-dma"),
    ("bfloat16", 1, 0, 4352, 4096, 4096, 1, 0, "gemm tn 256x256 lds-dma 16-bit split-tail 16x8"),
    # NN with more tiles than CUs: persistent tiles (split tail with a shared
    # final sum; unsplit with ragged edges; the C5 out-projection's dX shape)
    ("bfloat16", 0, 0, 4352, 4096, 4096, 1, 1, "gemm nn 256x256 lds-dma 16-bit persistent split-tail 16x8"),
    ("bfloat16", 0, 0, 2104, 8000, 512, 1, 3, "gemm nn 256x256 lds-dma 16-bit persistent"),
    ("bfloat16", 0, 0, 17776, 1920, 1920, 1, 1, "gemm nn 256x256 lds-dma 16-bit persistent split-tail 48x3"),
    ("float16", 0, 0, 4352, 4096, 4096, 1, 2, "gemm nn 256x256 lds-dma 16-bit persistent split-tail 16x8"),
    ("float16", 1, 0, 2104, 8000, 512, 1, 2, "gemm tn 256x256 lds-dma"),
    # weight-gradient shapes: few output tiles, long and ragged K (tokens)
    ("bfloat16", 1, 0, 1920, 1920, 4000, 1, 0, "gemm tn 256x256 lds-dma 16-bit split-tail 64x4"),
    ("bfloat16", 1, 0, 5760, 1920, 1000, 1, 0, "gemm tn 256x256 lds-dma"),
    ("float16", 1, 0, 1000, 1000, 1112, 1, 1, "gemm tn 256x256 lds-dma 16-bit split-tail 16x8"),
    ("bfloat16", 0, 0, 5760, 1920, 1024, 1, 0, "gemm nn 256x256 lds-dma"),
]


@pytest.mark.parametrize("case", LDS_DMA_CASES, ids=lambda c: "%s-%s%s-%dx%dx%dx%d-e%d" % (
    c[0], "T" if c[1] else "N", "T" if c[2] else "N", c[3], c[4], c[5], c[6], c[7]))
def test_lds_dma_layouts(case):
    """The 256x256 LDS-DMA kernel with M/N-contiguous operands (transposing
    fragment reads), ragged edges, batches, the split tail and epilogues,
    through the C ABI: sampled rows against fp64 plus row and column
    checksums of the whole output."""
    dtype, ta, tb, m, n, k, batch, epi, expect = case
    rng = np.random.default_rng(9000 + m + n + k + 10 * ta + tb + batch)
    shp = lambda *s: ((batch,) if batch > 1 else ()) + s  # noqa: E731
    a = rnd(rng, shp(k, m) if ta else shp(m, k), 1.0, dtype)
    b = rnd(rng, shp(n, k) if tb else shp(k, n), 1.0 / np.sqrt(k), dtype)
    bias = rnd(rng, (n,), 0.5, dtype)
    ga, gb, gbias = up(a, dtype), up(b, dtype), up(bias, dtype)
    lda, ldb = (m if ta else k), (k if tb else n)
    plan = cu().gemm_plan(tb, m, n, k, batch, ga.data_ptr, lda, m * k if batch > 1 else 0, gb.data_ptr, ldb,
                          n * k if batch > 1 else 0, n, m * n, ga.dtype, epi=epi,
                          ptr_bias=gbias.data_ptr if epi in (1, 2, 3) else 0, transA=ta)
    assert plan.startswith(expect), plan
    gc = cu().empty(shp(m, n), ga.dtype, 0)
    I64 = ctypes.c_int64
    lib = _lib()
    rc = lib.sf_gemm(ta, tb, I64(m), I64(n), I64(k), I64(batch), ctypes.c_void_p(ga.data_ptr), I64(lda),
                     I64(m * k if batch > 1 else 0), ctypes.c_void_p(gb.data_ptr), I64(ldb),
                     I64(n * k if batch > 1 else 0), ctypes.c_void_p(gc.data_ptr), I64(n), I64(m * n), SFD[dtype],
                     SFD[dtype], ctypes.c_float(1.0), ctypes.c_void_p(gbias.data_ptr if epi in (1, 2, 3) else None),
                     epi, None)
    assert rc == 0, lib.sf_last_error()
    cu().device_synchronize()
    y = down(gc).reshape(batch, m, n)
    a3 = a.reshape((batch, k, m) if ta else (batch, m, k)).astype(np.float64)
    b3 = b.reshape((batch, n, k) if tb else (batch, k, n)).astype(np.float64)
    am = np.swapaxes(a3, -2, -1) if ta else a3
    bm = np.swapaxes(b3, -2, -1) if tb else b3
    act = {0: None, 1: None, 2: "silu", 3: "gelu"}[epi]
    rows = np.unique(np.r_[0, m - 1, np.arange(0, m, 97), np.arange(255, m, 256), np.arange(256, m, 256)])
    for bi in sorted({0, batch - 1}):
        pre = am[bi, rows] @ bm[bi] + (bias.astype(np.float64) if epi else 0.0)
        y64 = ref.act_f64(pre, act)
        absprod = np.abs(am[bi, rows]) @ np.abs(bm[bi]) + (np.abs(bias.astype(np.float64)) if epi else 0.0)
        check_bound(y[bi, rows], y64, gemm_bound(y64, absprod, k, dtype, act), "%s rows" % (case,))
        if epi == 0:
            rs = y[bi].astype(np.float64).sum(axis=1)
            cs = y[bi].astype(np.float64).sum(axis=0)
            full_abs = np.abs(am[bi]) @ np.abs(bm[bi])
            eps = 2 * (k * 2.0 ** -23 + {"float16": 2.0 ** -11, "bfloat16": 2.0 ** -8}[dtype])
            assert np.all(np.abs(rs - am[bi] @ bm[bi].sum(axis=1)) <= eps * full_abs.sum(axis=1) + 1e-6)
            assert np.all(np.abs(cs - am[bi].sum(axis=0) @ bm[bi]) <= eps * full_abs.sum(axis=0) + 1e-6)


def test_lds_dma_split_tail_is_deterministic():
    rng = np.random.default_rng(31)
    m, n, k = 4352, 4096, 1024
    a = up(rnd(rng, (k, m), 1.0, "bfloat16"), "bfloat16")
    b = up(rnd(rng, (k, n), 0.03, "bfloat16"), "bfloat16")
    y1 = cu().gputensor_bits_to_numpy(cu().dev_matmul_tn(a, b))
    y2 = cu().gputensor_bits_to_numpy(cu().dev_matmul_tn(a, b))
    assert np.array_equal(y1, y2)
