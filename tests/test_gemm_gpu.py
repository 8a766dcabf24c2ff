"""GEMM parity on the GPU, small and ragged shapes: every tile config and
operand layout of sf_gemm against the fp64 closed form (and, for fp32,
against the reference's CPU fp32 path), through the Cython seam and the C
ABI."""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from helpers import check_bound, cu, down, gemm_bound, quantize, ref, rnd, up
from oracle.configs import normwise_err, tol_fp32

pytestmark = pytest.mark.gpu

DTYPES = ["float32", "float16", "bfloat16"]


def _case(rng, m, n, k, dtype, nt):
    a = rnd(rng, (m, k), 1.0, dtype)
    b = rnd(rng, (n, k) if nt else (k, n), 1.0 / np.sqrt(max(k, 1)), dtype)
    return a, b


def test_sgemm_known_answer_like_reference():
    """Mirror of the reference's only GEMM known-answer check
    (tests/test_mps_ops.py:24-33): seed 42, 3x4 @ 4x2, max error < 1e-5
    against NumPy."""
    np.random.seed(42)
    a = np.random.randn(3, 4).astype(np.float32)
    b = np.random.randn(4, 2).astype(np.float32)
    c = down(cu().dev_matmul(up(a, "float32"), up(b, "float32")))
    assert c.shape == (3, 2)
    assert np.max(np.abs(c - a @ b)) < 1e-5


SMALL = [(1, 1, 1), (3, 5, 7), (2, 3, 8), (5, 9, 16), (17, 33, 65), (64, 64, 64),
         (100, 130, 72), (129, 257, 200), (16, 48, 4096), (33, 40, 96), (7, 300, 1000),
         (255, 257, 128), (300, 64, 520)]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("nt", [False, True], ids=["NN", "NT"])
@pytest.mark.parametrize("shape", SMALL, ids=lambda s: "x".join(map(str, s)))
def test_gemm_small(dtype, nt, shape):
    m, n, k = shape
    rng = np.random.default_rng(1000 + m * 7 + n * 13 + k)
    a, b = _case(rng, m, n, k, dtype, nt)
    ga, gb = up(a, dtype), up(b, dtype)
    y = down(cu().dev_matmul_nt(ga, gb) if nt else cu().dev_matmul(ga, gb))
    bm = b.T if nt else b
    y64 = ref.matmul_f64(a, bm)
    absprod = np.abs(a.astype(np.float64)) @ np.abs(bm.astype(np.float64))
    assert y.shape == (m, n)
    check_bound(y, y64, gemm_bound(y64, absprod, k, dtype), "%s %s %s" % (dtype, nt, shape))
    if dtype == "float32":
        y_cpu = ref.matmul_nt(a, b) if nt else ref.matmul(a, b)
        assert normwise_err(y, y_cpu) <= tol_fp32(k)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("act", [None, "silu", "gelu"])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("shape", [(1, 40, 64), (16, 1000, 256), (3, 17, 24), (70, 200, 136),
                                   (300, 520, 264)], ids=lambda s: "x".join(map(str, s)))
def test_linear_epilogues(dtype, act, bias, shape):
    m, n, k = shape
    rng = np.random.default_rng(77 + m + n + k)
    x = rnd(rng, (m, k), 1.0, dtype)
    w = rnd(rng, (n, k), 1.0 / np.sqrt(k), dtype)
    b = rnd(rng, (n,), 0.5, dtype) if bias else None
    gb = up(b, dtype) if bias else None
    y = down(cu().dev_linear_forward(up(x, dtype), up(w, dtype), gb, act))
    y64 = ref.linear_f64(x, w, b, act)
    absprod = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    check_bound(y, y64, gemm_bound(y64, absprod, k, dtype, act), "linear %s %s %s" % (dtype, act, shape))


def test_linear_leading_dims_and_strides():
    """Output shape x.shape[:-1] + (N,), C-contiguous (reference
    _cuda_ops.pyx:1301)."""
    rng = np.random.default_rng(5)
    x = rnd(rng, (2, 3, 5, 64), 1.0, "bfloat16")
    w = rnd(rng, (24, 64), 0.1, "bfloat16")
    gy = cu().dev_linear_forward(up(x, "bfloat16"), up(w, "bfloat16"))
    assert gy.shape == (2, 3, 5, 24)
    y = down(gy)
    assert y.flags.c_contiguous and y.strides == (3 * 5 * 24 * 4, 5 * 24 * 4, 24 * 4, 4)
    y64 = ref.linear_f64(x.reshape(-1, 64), w).reshape(2, 3, 5, 24)
    absprod = (np.abs(x.reshape(-1, 64).astype(np.float64)) @ np.abs(w.astype(np.float64)).T).reshape(y64.shape)
    check_bound(y, y64, gemm_bound(y64, absprod, 64, "bfloat16"))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("nt", [False, True], ids=["NN", "NT"])
@pytest.mark.parametrize("bcast", ["none", "b2d", "a2d"])
def test_batched(dtype, nt, bcast):
    rng = np.random.default_rng(11)
    bshape, m, n, k = (2, 3), 40, 72, 48
    a_shape = (m, k) if bcast == "a2d" else bshape + (m, k)
    b_core = (n, k) if nt else (k, n)
    b_shape = b_core if bcast == "b2d" else bshape + b_core
    a = rnd(rng, a_shape, 1.0, dtype)
    b = rnd(rng, b_shape, 1.0 / np.sqrt(k), dtype)
    fn = cu().dev_batched_matmul_nt if nt else cu().dev_batched_matmul
    y = down(fn(up(a, dtype), up(b, dtype)))
    bm = np.swapaxes(b, -2, -1) if nt else b
    y64 = np.matmul(a.astype(np.float64), bm.astype(np.float64))
    absprod = np.matmul(np.abs(a.astype(np.float64)), np.abs(bm.astype(np.float64)))
    assert y.shape == bshape + (m, n)
    check_bound(y, y64, gemm_bound(y64, absprod, k, dtype), "batched %s %s %s" % (dtype, nt, bcast))


@pytest.mark.parametrize("bcast", ["b2d", "a2d"])
def test_batched_k64_broadcast(bcast):
    """Batched NT with K = 64 on the K = 64 kernel (128 x 128 tiles), one
    operand broadcast over the batch (batch stride 0), alpha-scaled as the
    attention scores are; every output against fp64."""
    rng = np.random.default_rng(13 + (bcast == "a2d"))
    bsz, m, n, k = 4, 1100, 1000, 64
    a = rnd(rng, (m, k) if bcast == "a2d" else (bsz, m, k), 1.0, "float16")
    b = rnd(rng, (n, k) if bcast == "b2d" else (bsz, n, k), 1.0, "float16")
    ga, gb = up(a, "float16"), up(b, "float16")
    plan = cu().gemm_plan(1, m, n, k, bsz, ga.data_ptr, k, 0 if bcast == "a2d" else m * k, gb.data_ptr, k,
                          0 if bcast == "b2d" else n * k, n, m * n, "float16")
    assert plan == "gemm nt 128x128 k64 lds-dma 16-bit", plan
    y = down(cu().dev_batched_matmul_nt(ga, gb, 0.125))
    bm = np.swapaxes(b, -2, -1)
    y64 = 0.125 * np.matmul(a.astype(np.float64), bm.astype(np.float64))
    absprod = 0.125 * np.matmul(np.abs(a.astype(np.float64)), np.abs(bm.astype(np.float64)))
    assert y.shape == (bsz, m, n)
    check_bound(y, y64, gemm_bound(y64, absprod, k, "float16"), "batched k64 %s" % bcast)


def test_batched_nt_alpha():
    rng = np.random.default_rng(12)
    q = rnd(rng, (4, 96, 64), 1.0, "float16")
    k = rnd(rng, (4, 80, 64), 1.0, "float16")
    s = down(cu().dev_batched_matmul_nt(up(q, "float16"), up(k, "float16"), 0.125))
    s64 = 0.125 * np.matmul(q.astype(np.float64), np.swapaxes(k, -2, -1).astype(np.float64))
    absprod = 0.125 * np.matmul(np.abs(q.astype(np.float64)), np.abs(np.swapaxes(k, -2, -1)).astype(np.float64))
    check_bound(s, s64, gemm_bound(s64, absprod, 64, "float16"))


# Shapes chosen so the dispatcher picks each tile config (asserted through
# sf_gemm_plan), checked on sampled rows plus row/column checksums.
TILE_CASES = [
    # (dtype, nt, M, N, K, batch, expected kernel)
    ("bfloat16", True, 4096, 4096, 192, 1, "gemm tile 256x256"),
    ("bfloat16", True, 4096, 4096, 256, 1, "gemm nt 256x256 lds-dma"),
    ("float16", True, 4000, 4100, 384, 1, "gemm nt 256x256 lds-dma"),
    ("bfloat16", True, 1000, 1100, 128, 16, "gemm nt 256x256 lds-dma"),
    ("float16", True, 2000, 2100, 64, 8, "gemm nt 128x128 k64 lds-dma"),
    ("bfloat16", True, 4096, 4096, 64, 1, "gemm nt 128x128 k64 lds-dma"),
    ("bfloat16", True, 1000, 4001, 64, 3, "gemm nt 128x128 k64 lds-dma"),
    ("bfloat16", False, 4096, 4096, 192, 1, "gemm tile 256x256"),
    ("float16", True, 2048, 4096, 136, 1, "gemm tile 256x128"),
    ("bfloat16", False, 2048, 4096, 136, 1, "gemm tile 256x128"),
    ("bfloat16", True, 2048, 2048, 200, 1, "gemm tile 128x128"),
    ("float16", False, 2048, 2048, 200, 1, "gemm tile 128x128"),
    ("float16", False, 4096, 64, 264, 16, "gemm tile 256x64"),
    ("bfloat16", True, 4096, 48, 264, 16, "gemm tile 256x64"),
    ("bfloat16", True, 300, 500, 256, 1, "gemm tile 64x64"),
    ("float16", True, 300, 500, 250, 1, "gemm tile generic"),
    ("bfloat16", False, 300, 500, 250, 1, "gemm tile generic"),
    ("bfloat16", True, 16, 11008, 4096, 1, "gemm skinny line"),
    ("bfloat16", True, 1, 11008, 4096, 1, "gemm skinny line"),
    ("float16", True, 3, 1000, 2048, 1, "gemm skinny line"),
    ("bfloat16", True, 7, 20001, 8192, 1, "gemm skinny line"),
    ("float16", True, 16, 37, 4096, 5, "gemm skinny line"),
    ("bfloat16", True, 2, 16389, 2048, 2, "gemm skinny line"),
    ("bfloat16", True, 16, 4000, 1920, 1, "gemm skinny"),
    ("float16", True, 5, 333, 1000, 3, "gemm skinny"),
    ("float32", True, 2048, 2048, 136, 1, "gemm tile 128x128"),
    ("float32", False, 2048, 2048, 136, 1, "gemm tile 128x128"),
    ("float32", False, 1000, 900, 100, 1, "gemm tile 64x64"),
    ("float32", True, 333, 270, 99, 1, "gemm tile generic"),
    ("float32", True, 64, 512, 512, 1, "gemm small 16x16"),
    ("float32", False, 50, 72, 300, 3, "gemm small 16x16"),
    ("float32", True, 200, 300, 1000, 1, "gemm small 16x32"),
    ("float32", False, 512, 512, 512, 1, "gemm small 16x32"),
    ("float32", False, 500, 508, 64, 2, "gemm tile 64x64 lds-dma k-groups"),
    ("float32", False, 1000, 900, 256, 1, "gemm tile 64x64 lds-dma k-groups"),
    ("float32", True, 1000, 900, 256, 1, "gemm tile 64x64 lds-dma k-groups"),
    ("float32", False, 2048, 2048, 2048, 1, "gemm tile 64x64 lds-dma k-groups"),
    ("float32", True, 300, 200, 160, 4, "gemm tile 64x64 lds-dma fp32"),
    ("float32", False, 300, 200, 160, 4, "gemm tile 64x64 lds-dma fp32"),
]


@pytest.mark.parametrize("case", TILE_CASES, ids=lambda c: "%s-%s-%dx%dx%dx%d" % (c[0], "NT" if c[1] else "NN", c[2], c[3], c[4], c[5]))
def test_tile_configs(case):
    dtype, nt, m, n, k, batch, expect = case
    rng = np.random.default_rng(m + 3 * n + 5 * k + batch)
    shp = lambda *s: ((batch,) if batch > 1 else ()) + s  # noqa: E731
    a = rnd(rng, shp(m, k), 1.0, dtype)
    b = rnd(rng, shp(n, k) if nt else shp(k, n), 1.0 / np.sqrt(k), dtype)
    ga, gb = up(a, dtype), up(b, dtype)
    ldb = k if nt else n
    plan = cu().gemm_plan(1 if nt else 0, m, n, k, batch, ga.data_ptr, k, m * k if batch > 1 else 0,
                          gb.data_ptr, ldb, n * k if batch > 1 else 0, n, m * n, ga.dtype)
    assert plan.startswith(expect), plan
    if batch > 1:
        fn = cu().dev_batched_matmul_nt if nt else cu().dev_batched_matmul
    else:
        fn = cu().dev_matmul_nt if nt else cu().dev_matmul
    y = down(fn(ga, gb)).reshape(batch, m, n)
    a3 = a.reshape(batch, m, k).astype(np.float64)
    b3 = b.reshape((batch, n, k) if nt else (batch, k, n)).astype(np.float64)
    bm = np.swapaxes(b3, -2, -1) if nt else b3
    rows = np.unique(np.r_[0, m - 1, np.arange(0, m, 97), np.arange(255, m, 256), np.arange(256, m, 256)])
    for bi in sorted({0, batch - 1}):
        y64 = a3[bi, rows] @ bm[bi]
        absprod = np.abs(a3[bi, rows]) @ np.abs(bm[bi])
        check_bound(y[bi, rows], y64, gemm_bound(y64, absprod, k, dtype), "%s rows" % (case,))
        # Checksums over every row and column of this batch entry.
        rs = y[bi].astype(np.float64).sum(axis=1)
        rs64 = a3[bi] @ bm[bi].sum(axis=1)
        cs = y[bi].astype(np.float64).sum(axis=0)
        cs64 = a3[bi].sum(axis=0) @ bm[bi]
        full_abs = np.abs(a3[bi]) @ np.abs(bm[bi])
        eps = 2 * (k * 2.0 ** -23 + {"float32": 2.0 ** -24, "float16": 2.0 ** -11, "bfloat16": 2.0 ** -8}[dtype])
        assert np.all(np.abs(rs - rs64) <= eps * full_abs.sum(axis=1) + 1e-6), "row checksum %s" % (case,)
        assert np.all(np.abs(cs - cs64) <= eps * full_abs.sum(axis=0) + 1e-6), "col checksum %s" % (case,)


@pytest.mark.parametrize("act,n", [(None, 8000), ("silu", 8000), ("gelu", 8000), ("silu", 7999), (None, 8191)])
def test_big_nt_linear_epilogues(act, n):
    """The 256x256 LDS-DMA NT kernel with bias and fused activations on ragged
    edges (M, N not tile multiples), checked on sampled rows and edge rows.
    An even N moves the tile's bias into LDS with its first k-pair; an odd N
    loads it in the epilogue."""
    m, k = 2100, 512
    rng = np.random.default_rng(31 + n)
    x = rnd(rng, (m, k), 1.0, "bfloat16")
    w = rnd(rng, (n, k), 1.0 / np.sqrt(k), "bfloat16")
    b = rnd(rng, (n,), 0.5, "bfloat16")
    gx, gw, gb = up(x, "bfloat16"), up(w, "bfloat16"), up(b, "bfloat16")
    plan = cu().gemm_plan(1, m, n, k, 1, gx.data_ptr, k, 0, gw.data_ptr, k, 0, n, 0, gx.dtype,
                          epi=1, ptr_bias=gb.data_ptr)
    assert plan.startswith("gemm nt 256x256 lds-dma"), plan
    y = down(cu().dev_linear_forward(gx, gw, gb, act))
    rows = np.unique(np.r_[0, 255, 256, 1023, 1024, 2047, 2048, m - 1, np.arange(3, m, 61)])
    y64 = ref.linear_f64(x[rows], w, b, act)
    absprod = np.abs(x[rows].astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    check_bound(y[rows], y64, gemm_bound(y64, absprod, k, "bfloat16", act), "big nt %s" % act)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("act,bias", [(None, False), (None, True), ("silu", True), ("gelu", False)])
@pytest.mark.parametrize("mn", [(2100, 4096), (1000, 4001)], ids=lambda s: "x".join(map(str, s)))
def test_k64_linear_epilogues(dtype, act, bias, mn):
    """The K = 64 kernel (128 x 128 tiles, four workgroups per CU) with and
    without bias and with fused activations, partial row and column tiles
    and an odd N; every output against fp64."""
    m, n = mn
    k = 64
    rng = np.random.default_rng(m + n + (act == "silu") + 2 * bias)
    x = rnd(rng, (m, k), 1.0, dtype)
    w = rnd(rng, (n, k), 1.0 / np.sqrt(k), dtype)
    b = rnd(rng, (n,), 0.5, dtype) if bias else None
    gx, gw = up(x, dtype), up(w, dtype)
    plan = cu().gemm_plan(1, m, n, k, 1, gx.data_ptr, k, 0, gw.data_ptr, k, 0, n, 0, gx.dtype,
                          epi=1 if bias else 0, ptr_bias=16 if bias else 0)
    assert plan == "gemm nt 128x128 k64 lds-dma 16-bit", plan
    y = down(cu().dev_linear_forward(gx, gw, up(b, dtype) if bias else None, act))
    y64 = ref.linear_f64(x, w, b, act)
    absprod = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    check_bound(y, y64, gemm_bound(y64, absprod, k, dtype, act), "k64 %s %s" % (act, bias))


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("act", [None, "silu", "gelu"])
@pytest.mark.parametrize("mnk", [(1, 11008, 4096), (16, 4099, 2048), (9, 700, 8192), (12, 5000, 4096),
                                 (8, 3001, 4096)],
                         ids=lambda s: "x".join(map(str, s)))
def test_skinny_line_linear_epilogues(dtype, act, mnk):
    """The row-segment skinny stream (K = 512 x waves) with bias and fused
    activations: every output checked, N not a multiple of 16 or of the
    rows per workgroup; M of 9-16 takes x in whole lines through LDS, M of
    at most 8 in the MFMA layout."""
    m, n, k = mnk
    rng = np.random.default_rng(m * 7 + n + k)
    x = rnd(rng, (m, k), 1.0, dtype)
    w = rnd(rng, (n, k), 1.0 / np.sqrt(k), dtype)
    b = rnd(rng, (n,), 0.5, dtype)
    gx, gw, gb = up(x, dtype), up(w, dtype), up(b, dtype)
    plan = cu().gemm_plan(1, m, n, k, 1, gx.data_ptr, k, 0, gw.data_ptr, k, 0, n, 0, gx.dtype,
                          epi=1, ptr_bias=gb.data_ptr)
    assert plan.startswith("gemm skinny line"), plan
    y = down(cu().dev_linear_forward(gx, gw, gb, act))
    y64 = ref.linear_f64(x, w, b, act)
    absprod = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    check_bound(y, y64, gemm_bound(y64, absprod, k, dtype, act), "skinny line %s %s %s" % (dtype, act, mnk))


@pytest.mark.parametrize("m", [4, 13])
def test_skinny_line_fp32_output(m):
    """16-bit inputs with an fp32 result through the row-segment stream."""
    n, k = 3000, 4096
    rng = np.random.default_rng(5)
    a = rnd(rng, (m, k), 1.0, "bfloat16")
    w = rnd(rng, (n, k), 1.0 / np.sqrt(k), "bfloat16")
    ga, gw = up(a, "bfloat16"), up(w, "bfloat16")
    out = cu().empty((m, n), np.float32, 0)
    plan = cu().gemm_plan(1, m, n, k, 1, ga.data_ptr, k, 0, gw.data_ptr, k, 0, n, 0, ga.dtype)
    assert plan.startswith("gemm skinny line"), plan
    so = ctypes.CDLL(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                  "scaffolding_amd", "libsfgemm.so"))
    I64, P = ctypes.c_int64, ctypes.c_void_p
    rc = so.sf_gemm(0, 1, I64(m), I64(n), I64(k), I64(1), P(ga.data_ptr), I64(k), I64(0), P(gw.data_ptr),
                    I64(k), I64(0), P(out.data_ptr), I64(n), I64(0), 2, 0, ctypes.c_float(1.0), None, 0, None)
    assert rc == 0
    cu().device_synchronize()
    y = down(out)
    y64 = a.astype(np.float64) @ w.astype(np.float64).T
    absprod = np.abs(a.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    check_bound(y, y64, gemm_bound(y64, absprod, k, "float32"), "skinny line fp32 out")


SPLIT_CASES = [
    # (M, N, K, act, bias, expected "split-tail R x s")
    (4352, 4096, 4096, None, False, "split-tail 16x8"),    # 272 tiles: 16 left over, 8 parts of 4 units
    (7900, 2800, 4352, "gelu", True, "split-tail 85x2"),  # 341 tiles: 85 left, 34 units in 2 parts (XCD packing)
    (17776, 1920, 7680, None, True, "split-tail 48x5"),   # C5 MLP-down shape
    (17776, 1920, 1920, "gelu", True, "split-tail 48x3"),  # C5 out-projection: short launch, 5 units a part
    # persistent tiles without a split: 2 rounds + 15 tiles; two whole rounds
    (4352, 7936, 1024, "silu", True, "persistent"),
    (4096, 8192, 512, None, True, "persistent"),
]


def test_persistent_split_off_xcd_fallback():
    """The persistent split tail places every part of a tile on one XCD and
    hands partials over through that XCD's L2.  A part that finds itself on
    another XCD (hardware XCC_ID) releases at agent scope and makes the last
    part acquire.  The xcd_shift test hook makes every part expect a different XCD,
    so all of them take that fallback: the output must be bit-identical to
    the same-XCD hand-off (same parts, same summation order)."""
    m, n, k = 4352, 4096, 4096
    rng = np.random.default_rng(77)
    x = rnd(rng, (m, k), 1.0, "bfloat16")
    w = rnd(rng, (n, k), 1.0 / np.sqrt(k), "bfloat16")
    gx, gw = up(x, "bfloat16"), up(w, "bfloat16")
    plan = cu().gemm_plan(1, m, n, k, 1, gx.data_ptr, k, 0, gw.data_ptr, k, 0, n, 0, gx.dtype)
    assert plan.endswith("persistent split-tail 16x8"), plan
    y0 = down(cu().dev_linear_forward(gx, gw, None))
    cu()._set_test_hooks(xcd_shift=3)
    try:
        y1 = down(cu().dev_linear_forward(gx, gw, None))
        y2 = down(cu().dev_linear_forward(gx, gw, None))
    finally:
        cu()._set_test_hooks()
    y3 = down(cu().dev_linear_forward(gx, gw, None))
    for y in (y1, y2, y3):
        assert np.array_equal(y.view(np.uint32), y0.view(np.uint32)), "fallback hand-off changed the output"
    rows = np.r_[0, 1000, m - 256, m - 1]
    y64 = ref.linear_f64(x[rows], w, None, None)
    absprod = np.abs(x[rows].astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    check_bound(y0[rows], y64, gemm_bound(y64, absprod, k, "bfloat16", None), "persistent split")


def test_persistent_split_shared_sum_sweep():
    """The parts of a persistent split tile share the final sum: each waits
    (a bounded number of polls) for the others, claims its slice of the rows
    and sums it; the last part to arrive takes every slice still unclaimed.
    The split_spins=0 test hook makes every part but the last give up at once, so
    the last part sums every slice: the output must be bit-identical (same
    partials, same part order), and the per-tile words must be back at zero
    for the next launch with the normal wait."""
    m, n, k = 4352, 4096, 4096
    rng = np.random.default_rng(78)
    x = rnd(rng, (m, k), 1.0, "bfloat16")
    w = rnd(rng, (n, k), 1.0 / np.sqrt(k), "bfloat16")
    b = rnd(rng, (n,), 0.5, "bfloat16")
    gx, gw, gb = up(x, "bfloat16"), up(w, "bfloat16"), up(b, "bfloat16")
    plan = cu().gemm_plan(1, m, n, k, 1, gx.data_ptr, k, 0, gw.data_ptr, k, 0, n, 0, gx.dtype)
    assert plan.endswith("persistent split-tail 16x8"), plan
    y0 = down(cu().dev_linear_forward(gx, gw, gb, "silu"))
    cu()._set_test_hooks(split_spins=0)
    try:
        y1 = down(cu().dev_linear_forward(gx, gw, gb, "silu"))
        y2 = down(cu().dev_linear_forward(gx, gw, gb, "silu"))
    finally:
        cu()._set_test_hooks()
    y3 = down(cu().dev_linear_forward(gx, gw, gb, "silu"))
    for y in (y1, y2, y3):
        assert np.array_equal(y.view(np.uint32), y0.view(np.uint32)), "the last-part sweep changed the output"
    rows = np.r_[0, 1000, m - 256, m - 129, m - 1]
    y64 = ref.linear_f64(x[rows], w, b, "silu")
    absprod = np.abs(x[rows].astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    check_bound(y0[rows], y64, gemm_bound(y64, absprod, k, "bfloat16", "silu"), "shared split sum")


def test_shared_split_sum_beside_another_kernel():
    """The shared split sum waits (bounded) for parts that are resident
    together in a persistent grid.  A persistent GEMM on a second stream,
    launched at the same time, holds CUs while the split launch runs, so some
    parts may start late: their siblings' waits run out and the last part
    sums the slices they left.  Either way both outputs must equal the ones
    computed alone, bit for bit."""
    so = ctypes.CDLL(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                  "scaffolding_amd", "libsfgemm.so"))
    I64, P = ctypes.c_int64, ctypes.c_void_p
    rng = np.random.default_rng(79)
    shapes = [(4352, 4096, 4096), (4096, 8192, 512)]  # split-tail 16x8; persistent, no split
    ops = []
    for (m, n, k), expect in zip(shapes, ("persistent split-tail 16x8", "persistent")):
        gx = up(rnd(rng, (m, k), 1.0, "bfloat16"), "bfloat16")
        gw = up(rnd(rng, (n, k), 1.0 / np.sqrt(k), "bfloat16"), "bfloat16")
        plan = cu().gemm_plan(1, m, n, k, 1, gx.data_ptr, k, 0, gw.data_ptr, k, 0, n, 0, gx.dtype)
        assert plan.endswith(expect), plan
        ops.append((m, n, k, gx, gw, cu().empty((m, n), cu().BFLOAT16)))
    cu().device_synchronize()
    streams = []
    for _ in range(2):
        sp = ctypes.c_void_p()
        assert so.sf_stream_create(ctypes.byref(sp)) == 0
        streams.append(sp)

    def gemm(i):
        m, n, k, gx, gw, out = ops[i]
        return so.sf_gemm(0, 1, I64(m), I64(n), I64(k), I64(1), P(gx.data_ptr), I64(k), I64(0), P(gw.data_ptr),
                          I64(k), I64(0), P(out.data_ptr), I64(n), I64(0), 2, 2, ctypes.c_float(1.0), None, 0,
                          streams[i])
    try:
        want = []
        for i in range(2):
            assert gemm(i) == 0 and so.sf_stream_synchronize(streams[i]) == 0
            want.append(cu().gputensor_bits_to_numpy(ops[i][5]).copy())
        for _ in range(30):
            assert gemm(1) == 0
            assert gemm(0) == 0
        for sp in streams:
            assert so.sf_stream_synchronize(sp) == 0
        for i in range(2):
            assert np.array_equal(cu().gputensor_bits_to_numpy(ops[i][5]), want[i]), "stream %d" % i
        # the per-tile words are back at zero: a later launch alone still matches
        assert gemm(0) == 0 and so.sf_stream_synchronize(streams[0]) == 0
        assert np.array_equal(cu().gputensor_bits_to_numpy(ops[0][5]), want[0])
    finally:
        for sp in streams:
            so.sf_stream_destroy(sp)


@pytest.mark.parametrize("case", SPLIT_CASES, ids=lambda c: "%dx%dx%d" % c[:3])
def test_split_tail_linear(case):
    """The 256x256 NT kernel with its last partial wave of tiles split over k:
    fp32 partials in a workspace, summed in part order (one workgroup per
    tile: by the last part; persistent tiles: the parts of a tile on one XCD,
    each summing and storing its slice of the rows); and persistent tiles
    without a split.
    Two launches in a row check that the per-tile counters reset; sampled
    rows (including every split tile's rows) against fp64, checksums over all."""
    m, n, k, act, bias, expect = case
    rng = np.random.default_rng(m + n + k)
    x = rnd(rng, (m, k), 1.0, "bfloat16")
    w = rnd(rng, (n, k), 1.0 / np.sqrt(k), "bfloat16")
    b = rnd(rng, (n,), 0.5, "bfloat16") if bias else None
    gx, gw = up(x, "bfloat16"), up(w, "bfloat16")
    gb = up(b, "bfloat16") if bias else None
    plan = cu().gemm_plan(1, m, n, k, 1, gx.data_ptr, k, 0, gw.data_ptr, k, 0, n, 0, gx.dtype,
                          epi=1 if bias else 0, ptr_bias=gb.data_ptr if bias else 0)
    assert plan.startswith("gemm nt 256x256 lds-dma") and expect in plan, plan
    y1 = down(cu().dev_linear_forward(gx, gw, gb, act))
    y2 = down(cu().dev_linear_forward(gx, gw, gb, act))
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32)), "split tail not deterministic"
    # rows of the last tile rows (where split tiles sit in tile order) and a sample
    rows = np.unique(np.r_[0, m - 1, np.arange(0, m, 131), np.arange(max(0, m - 600), m, 7)])
    y64 = ref.linear_f64(x[rows], w, b, act)
    absprod = np.abs(x[rows].astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    check_bound(y1[rows], y64, gemm_bound(y64, absprod, k, "bfloat16", act), "split tail %s" % (case,))
    if act is None:
        rs64 = x.astype(np.float64) @ w.astype(np.float64).sum(axis=0)
        if bias:
            rs64 = rs64 + b.astype(np.float64).sum()
        full = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).sum(axis=0)
        eps = 2 * (k * 2.0 ** -23 + 2.0 ** -8)
        assert np.all(np.abs(y1.astype(np.float64).sum(axis=1) - rs64) <= eps * (full + n) + 1e-6)


def test_k_zero_writes_epilogue_of_zero():
    x = np.zeros((5, 0), np.float32)
    w = np.zeros((7, 0), np.float32)
    b = np.linspace(-1, 1, 7).astype(np.float32)
    y = down(cu().dev_linear_forward(up(x, "float32"), up(w, "float32"), up(b, "float32"), "silu"))
    np.testing.assert_allclose(y, np.broadcast_to(ref.silu(b.astype(np.float64)), (5, 7)), rtol=1e-6, atol=1e-7)


def test_empty_outputs():
    g = cu()
    y = g.dev_matmul(up(np.zeros((0, 4), np.float32), "float32"), up(np.zeros((4, 3), np.float32), "float32"))
    assert y.shape == (0, 3)
    y = g.dev_linear_forward(up(np.zeros((4, 8), np.float32), "bfloat16"), up(np.zeros((0, 8), np.float32), "bfloat16"))
    assert y.shape == (4, 0)


def test_shape_errors():
    g = cu()
    a = up(np.zeros((4, 8), np.float32), "float32")
    b = up(np.zeros((9, 3), np.float32), "float32")
    with pytest.raises(ValueError):
        g.dev_matmul(a, b)
    with pytest.raises(TypeError):
        g.dev_matmul(a, up(np.zeros((8, 3), np.float32), "bfloat16"))
    with pytest.raises(ValueError):
        g.dev_linear_forward(a, up(np.zeros((3, 7), np.float32), "float32"))


FP32_SPLIT = [
    # (M, N, K, transB, expected plan)
    (64, 4096, 4096, True, "gemm tile 64x64 lds-dma fp32 split-tail 64x4"),
    (200, 300, 4096, False, "gemm tile 64x64 lds-dma fp32 split-tail 20x8"),
    (100, 1000, 2560, True, "gemm tile 64x64 lds-dma fp32 split-tail 32x8"),
    (500, 700, 3000, False, "gemm tile 128x128 fp32 split-tail 24x8"),
    (300, 260, 3000, True, "gemm tile 64x64 fp32 split-tail 25x8"),
    # not split, checked the same way (run-to-run bit identity included)
    (64, 512, 512, True, "gemm small 16x16 fp32"),
    (768, 768, 1024, False, "gemm tile 64x64 lds-dma k-groups fp32"),
]


@pytest.mark.parametrize("case", FP32_SPLIT, ids=lambda c: "%dx%dx%d-%s" % (c[0], c[1], c[2], "NT" if c[3] else "NN"))
def test_fp32_split_k(case):
    """fp32 GEMMs with fewer tiles than CUs split every tile along k; the
    last part adds the partials in part order: checked elementwise against
    fp64 and the fp32 CPU path, and bit-identical across two runs."""
    m, n, k, nt, expect = case
    rng = np.random.default_rng(m + n + k)
    a = rnd(rng, (m, k), 1.0, "float32")
    b = rnd(rng, (n, k) if nt else (k, n), 1.0 / np.sqrt(k), "float32")
    ga, gb = up(a, "float32"), up(b, "float32")
    plan = cu().gemm_plan(1 if nt else 0, m, n, k, 1, ga.data_ptr, k, 0, gb.data_ptr, k if nt else n, 0, n, 0,
                          ga.dtype)
    assert plan == expect, plan
    fn = cu().dev_matmul_nt if nt else cu().dev_matmul
    y1 = fn(ga, gb)
    y2 = fn(ga, gb)
    assert np.array_equal(cu().gputensor_to_numpy(y1), cu().gputensor_to_numpy(y2))
    y = down(y1)
    bm = (b.T if nt else b).astype(np.float64)
    y64 = a.astype(np.float64) @ bm
    absprod = np.abs(a.astype(np.float64)) @ np.abs(bm)
    check_bound(y, y64, gemm_bound(y64, absprod, k, "float32"), "fp32 split %s" % (case,))
    y_cpu = ref.matmul_nt(a, b) if nt else ref.matmul(a, b)
    assert normwise_err(y, y_cpu) <= tol_fp32(k)
