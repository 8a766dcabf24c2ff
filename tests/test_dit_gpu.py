"""The DiT-block glue on the GPU (reference diffusion/models.py:470-590):
layer / RMS norm with the fused adaptive modulation, the residual fused
into every GEMM kernel, attention over heads read in place from packed
projections (ragged key counts included), the elementwise add, and the
whole block against the oracle (oracle/dit.py) — through the Cython seam
and the C ABI."""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from helpers import check_bound, cu, down, gemm_bound, out_half_ulp_rel, quantize, ref, rnd, up
from oracle import dit
from oracle.configs import normwise_err

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DTYPES = ["float32", "float16", "bfloat16"]


def _lib():
    so = ctypes.CDLL(os.path.join(ROOT, "scaffolding_amd", "libsfgemm.so"))
    so.sf_last_error.restype = ctypes.c_char_p
    return so


def norm_bound(y64, dtype):
    """One rounding into dtype plus the fp32 arithmetic of the row (mean,
    variance, rsqrt: a few 1e-6 relative of the normalised values)."""
    return (out_half_ulp_rel(dtype) + 2e-6) * np.abs(y64) + 2e-5 * (1.0 + np.abs(y64))


# ------------------------------------------------------------------ norms

NORM_SHAPES = [(1, 1), (3, 5), (7, 64), (33, 1920), (5, 4096), (2, 5000), (9, 200)]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("affine", [False, True], ids=["plain", "affine"])
@pytest.mark.parametrize("shape", NORM_SHAPES, ids=lambda s: "%dx%d" % s)
def test_layer_norm(dtype, affine, shape):
    r, c = shape
    rng = np.random.default_rng(r * 31 + c)
    x = quantize((rng.standard_normal((r, c)) * 2 + rng.standard_normal((r, 1))).astype(np.float32), dtype)
    g = rnd(rng, (c,), 1.0, dtype) if affine else None
    b = rnd(rng, (c,), 0.5, dtype) if affine else None
    y = down(cu().dev_layer_norm(up(x, dtype), up(g, dtype) if affine else None,
                                 up(b, dtype) if affine else None, 1e-5))
    y64 = dit.layer_norm_f64(x, g, b, 1e-5)
    check_bound(y, y64, norm_bound(y64, dtype), "layer_norm %s %s" % (dtype, shape))
    if dtype == "float32":
        y_ref = dit.layer_norm(x, g, b, 1e-5) if affine else dit.layer_norm(x, eps=1e-5)
        assert normwise_err(y, y_ref) <= 1e-5


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(2, 5, 64), (3, 7, 1920), (1, 300, 128), (2, 3, 37)],
                         ids=lambda s: "x".join(map(str, s)))
def test_ada_layer_norm(dtype, shape):
    """Fused LayerNorm + h (1 + scale) + shift with one modulation row per
    batch entry, read from one packed (B, 2C) projection."""
    bsz, n, c = shape
    rng = np.random.default_rng(bsz * 100 + n + c)
    x = rnd(rng, shape, 1.5, dtype)
    g, b = rnd(rng, (c,), 1.0, dtype), rnd(rng, (c,), 0.3, dtype)
    params = rnd(rng, (bsz, 2 * c), 0.4, dtype)
    y = down(cu().dev_ada_layer_norm(up(x, dtype), up(params, dtype), 1e-5, up(g, dtype), up(b, dtype)))
    y64 = dit.layer_norm_f64(x, g, b, 1e-5, params[:, None, :c], params[:, None, c:])
    check_bound(y, y64, norm_bound(y64, dtype) * 1.5, "ada_layer_norm %s %s" % (dtype, shape))
    # (B, 1, 2C) params: the same rows
    y2 = down(cu().dev_ada_layer_norm(up(x, dtype), up(params.reshape(bsz, 1, 2 * c), dtype), 1e-5,
                                      up(g, dtype), up(b, dtype)))
    assert np.array_equal(y, y2)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", NORM_SHAPES, ids=lambda s: "%dx%d" % s)
def test_rms_norm(dtype, shape):
    r, c = shape
    rng = np.random.default_rng(r + 17 * c)
    x = rnd(rng, (r, c), 2.0, dtype)
    g = rnd(rng, (c,), 1.0, dtype)
    y = down(cu().dev_rms_norm(up(x, dtype), up(g, dtype), 1e-6))
    y64 = dit.rms_norm_f64(x, g, 1e-6)
    check_bound(y, y64, norm_bound(y64, dtype), "rms_norm %s %s" % (dtype, shape))


def test_layer_norm_abi_stats_and_in_place():
    """mean_out / rstd_out through the C ABI, x == y in place, and the
    argument checks."""
    so = _lib()
    rng = np.random.default_rng(5)
    x = rnd(rng, (6, 96), 3.0, "float32") + 2
    gx = up(x, "float32")
    stats = up(np.zeros(12, np.float32), "float32")
    P, I64 = ctypes.c_void_p, ctypes.c_int64
    base = stats.data_ptr
    rc = so.sf_layer_norm(P(gx.data_ptr), P(gx.data_ptr), I64(6), I64(96), None, None, ctypes.c_float(1e-5),
                          None, None, I64(0), I64(1), P(base), P(base + 24), 0, None)
    assert rc == 0, so.sf_last_error()
    cu().device_synchronize()
    st = down(stats)
    x64 = x.astype(np.float64)
    np.testing.assert_allclose(st[:6], x64.mean(axis=1), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(st[6:], 1 / np.sqrt(x64.var(axis=1) + 1e-5), rtol=1e-5)
    y64 = dit.layer_norm_f64(x, eps=1e-5)
    check_bound(down(gx), y64, norm_bound(y64, "float32"), "in place")
    bad = so.sf_layer_norm(P(gx.data_ptr), P(gx.data_ptr), I64(6), I64(0), None, None, ctypes.c_float(1e-5),
                           None, None, I64(0), I64(1), None, None, 0, None)
    assert bad == -2
    bad = so.sf_layer_norm(P(gx.data_ptr), P(gx.data_ptr), I64(6), I64(96), None, None, ctypes.c_float(1e-5),
                           P(gx.data_ptr), None, I64(10), I64(1), None, None, 0, None)
    assert bad == -2 and b"mod_ld" in so.sf_last_error()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [1, 7, 8, 1000, 123457])
def test_add_bit_exact(dtype, n):
    rng = np.random.default_rng(n)
    a, b = rnd(rng, (n,), 1.0, dtype), rnd(rng, (n,), 1.0, dtype)
    y = down(cu().dev_add(up(a, dtype), up(b, dtype)))
    want = quantize(a.astype(np.float32) + b.astype(np.float32), dtype)
    assert np.array_equal(y, want)


# ------------------------------------------------------------------ residual GEMM

RES_CASES = [  # (dtype, m, n, k, kernel name prefix)
    ("bfloat16", 1, 40, 64, "gemm skinny"),
    ("bfloat16", 4, 300, 2048, "gemm skinny line"),
    ("float16", 70, 200, 136, "gemm tile"),
    ("bfloat16", 300, 520, 264, "gemm tile"),
    ("bfloat16", 4096, 4096, 128, "gemm nt 256x256 lds-dma"),
    ("float16", 2100, 4001, 64, "gemm nt 128x128 k64 lds-dma"),  # K = 64: four workgroups per CU
    ("bfloat16", 4352, 4096, 4096, "gemm nt 256x256 lds-dma 16-bit persistent split"),  # split tail
    ("float16", 4352, 7936, 256, "gemm nt 256x256 lds-dma 16-bit persistent"),  # 527 tiles, persistent
    ("float32", 70, 200, 136, "gemm small 16x16"),
    ("float32", 64, 64, 1024, "gemm small 16x16"),
    ("float32", 5, 33, 20, "gemm small 16x16"),
    ("float32", 200, 300, 1000, "gemm small 16x32"),
    ("float32", 600, 520, 256, "gemm tile 64x64 lds-dma k-groups"),
    ("float32", 600, 520, 160, "gemm tile 64x64 lds-dma fp32"),           # odd slice count: one k-group
    ("float32", 64, 1000, 4096, "gemm tile 64x64 lds-dma fp32 split"),    # fp32 split-K
    ("float32", 70, 200, 4004, "gemm tile 64x64 fp32 split"),             # K % 32 != 0: register-staged
]


@pytest.mark.parametrize("case", RES_CASES, ids=lambda c: "%s-%dx%dx%d" % c[:4])
@pytest.mark.parametrize("act", [None, "silu"])
def test_linear_residual_every_kernel(case, act):
    dtype, m, n, k, kern = case
    rng = np.random.default_rng(m + 3 * n + 7 * k)
    x = rnd(rng, (m, k), 1.0, dtype)
    w = rnd(rng, (n, k), 1.0 / np.sqrt(k), dtype)
    b = rnd(rng, (n,), 0.5, dtype)
    r = rnd(rng, (m, n), 1.0, dtype)
    g = cu()
    gx, gw = up(x, dtype), up(w, dtype)
    plan = g.gemm_plan(1, m, n, k, 1, gx.data_ptr, k, 0, gw.data_ptr, k, 0, n, m * n, dtype, epi=1, ptr_bias=16)
    assert plan.startswith(kern), plan
    y = down(g.dev_linear_forward(gx, gw, up(b, dtype), act, up(r, dtype)))
    y64 = ref.linear_f64(x, w, b, act) + r.astype(np.float64)
    absprod = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    check_bound(y, y64, gemm_bound(y64, absprod, k, dtype, act), "residual %s %s" % (case, act))


def test_gemm_add_in_place_and_batched():
    """R == C (in-place accumulate) through the C ABI, and a batched NN
    product with a broadcast residual (strideR 0)."""
    so = _lib()
    g = cu()
    rng = np.random.default_rng(11)
    m, n, k = 300, 260, 192
    a, bt = rnd(rng, (m, k), 1.0, "bfloat16"), rnd(rng, (n, k), 0.1, "bfloat16")
    c0 = rnd(rng, (m, n), 1.0, "bfloat16")
    ga, gb, gc = up(a, "bfloat16"), up(bt, "bfloat16"), up(c0, "bfloat16")
    P, I64 = ctypes.c_void_p, ctypes.c_int64
    rc = so.sf_gemm_add(0, 1, I64(m), I64(n), I64(k), I64(1), P(ga.data_ptr), I64(k), I64(0), P(gb.data_ptr),
                        I64(k), I64(0), P(gc.data_ptr), I64(n), I64(0), 2, 2, ctypes.c_float(1.0), None, 0,
                        P(gc.data_ptr), I64(n), I64(0), None)
    assert rc == 0, so.sf_last_error()
    y64 = ref.matmul_f64(a, bt.T) + c0.astype(np.float64)
    absprod = np.abs(a.astype(np.float64)) @ np.abs(bt.astype(np.float64)).T
    check_bound(down(gc), y64, gemm_bound(y64, absprod, k, "bfloat16"), "in place")
    # R == C with a different ldr is refused
    rc = so.sf_gemm_add(0, 1, I64(m), I64(n), I64(k), I64(1), P(ga.data_ptr), I64(k), I64(0), P(gb.data_ptr),
                        I64(k), I64(0), P(gc.data_ptr), I64(n), I64(0), 2, 2, ctypes.c_float(1.0), None, 0,
                        P(gc.data_ptr), I64(n + 8), I64(0), None)
    assert rc == -2
    # batched NN, residual broadcast over the batch
    bsz, m, n, k = 3, 70, 64, 96
    a = rnd(rng, (bsz, m, k), 1.0, "float16")
    bb = rnd(rng, (bsz, k, n), 0.1, "float16")
    r = rnd(rng, (m, n), 1.0, "float16")
    ga, gb, gr = up(a, "float16"), up(bb, "float16"), up(r, "float16")
    out = g.empty((bsz, m, n), np.float16)
    rc = so.sf_gemm_add(0, 0, I64(m), I64(n), I64(k), I64(bsz), P(ga.data_ptr), I64(k), I64(m * k),
                        P(gb.data_ptr), I64(n), I64(k * n), P(out.data_ptr), I64(n), I64(m * n), 1, 1,
                        ctypes.c_float(0.5), None, 0, P(gr.data_ptr), I64(n), I64(0), None)
    assert rc == 0, so.sf_last_error()
    y64 = 0.5 * ref.matmul_f64(a, bb) + r.astype(np.float64)
    absprod = 0.5 * np.abs(a.astype(np.float64)) @ np.abs(bb.astype(np.float64))
    check_bound(down(out), y64, gemm_bound(y64, absprod, k, "float16"), "batched broadcast residual")


@pytest.mark.parametrize("case", [
    ("bfloat16", 4096, 4096, 128, "gemm nt 256x256 lds-dma"),
    ("bfloat16", 4352, 4096, 4096, "gemm nt 256x256 lds-dma 16-bit persistent split"),
    ("float16", 4352, 7936, 256, "gemm nt 256x256 lds-dma 16-bit persistent"),
    ("bfloat16", 17776, 1920, 1920, "gemm nt 256x256 lds-dma 16-bit persistent split"),
], ids=lambda c: "%s-%dx%dx%d" % c[:4])
def test_gemm_add_in_place_bitwise_8wave(case):
    """The 8-wave kernel loads each epilogue pass's residual one pass ahead
    of its stores: with R == C (the residual accumulated in place) every
    element must still be read before it is overwritten, so the in-place
    result equals the out-of-place one bit for bit, whole tiles, persistent
    tiles and the split tail's shared final sum (parts storing only their
    own rows) alike.  Ragged M and N edges included (17776 rows, N = 7936)."""
    dtype, m, n, k, kern = case
    so = _lib()
    g = cu()
    rng = np.random.default_rng(m + n + k)
    x = rnd(rng, (m, k), 1.0, dtype)
    w = rnd(rng, (n, k), 1.0 / np.sqrt(k), dtype)
    bias = rnd(rng, (n,), 0.5, dtype)
    r = rnd(rng, (m, n), 1.0, dtype)
    gx, gw, gbias = up(x, dtype), up(w, dtype), up(bias, dtype)
    plan = g.gemm_plan(1, m, n, k, 1, gx.data_ptr, k, 0, gw.data_ptr, k, 0, n, m * n, dtype, epi=1, ptr_bias=16)
    assert plan.startswith(kern), plan
    dt = 1 if dtype == "float16" else 2
    P, I64 = ctypes.c_void_p, ctypes.c_int64
    outs = []
    for in_place in (False, True):
        gr = up(r, dtype)
        gc = gr if in_place else g.empty((m, n), gr.dtype)
        rc = so.sf_gemm_add(0, 1, I64(m), I64(n), I64(k), I64(1), P(gx.data_ptr), I64(k), I64(0),
                            P(gw.data_ptr), I64(k), I64(0), P(gc.data_ptr), I64(n), I64(0), dt, dt,
                            ctypes.c_float(1.0), P(gbias.data_ptr), 1, P(gr.data_ptr), I64(n), I64(0), None)
        assert rc == 0, so.sf_last_error()
        outs.append(g.gputensor_bits_to_numpy(gc))
    assert np.array_equal(outs[0], outs[1])
    # sampled rows (both ends, the ragged last tile) against fp64
    rows = np.unique(np.r_[0, m - 1, m - 2, np.arange(0, m, 997), np.arange(max(0, m - 300), m, 37)])
    y = down(g.dev_linear_forward(gx, gw, gbias, None, up(r, dtype)))[rows]
    y64 = ref.linear_f64(x[rows], w, bias) + r[rows].astype(np.float64)
    absprod = np.abs(x[rows].astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    check_bound(y, y64, gemm_bound(y64, absprod, k, dtype), "residual in place %s" % (case,))


# ------------------------------------------------------------------ attention over packed heads

def attn_bound(v, dtype, sk):
    eps = {"float16": 2.0 ** -11, "bfloat16": 2.0 ** -8, "float32": 2.0 ** -23}[dtype]
    vmax = float(np.max(np.abs(v)))
    return 2e-2 * np.sqrt(sk / 1024) + 3 * eps * vmax + 1e-6


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("shape", [(2, 100, 3), (1, 300, 2), (3, 1, 1), (1, 64, 4), (2, 129, 2), (1, 17, 30)],
                         ids=lambda s: "x".join(map(str, s)))
def test_attention_packed_in_place(dtype, shape):
    bsz, n, heads = shape
    c = heads * 64
    rng = np.random.default_rng(bsz + n + heads)
    qkv = rnd(rng, (bsz, n, 3 * c), 1.0, dtype)
    o = down(cu().dev_attention_packed(up(qkv, dtype), heads))
    o64 = dit.mha_f64(qkv[..., :c], qkv[..., c:2 * c], qkv[..., 2 * c:], heads)
    assert o.shape == (bsz, n, c)
    assert float(np.max(np.abs(o - o64))) <= attn_bound(qkv, dtype, n)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("shape", [(2, 100, 3, 32), (1, 129, 2, 16), (1, 70, 5, 48)],
                         ids=lambda s: "x".join(map(str, s)))
def test_attention_packed_small_head_sizes(dtype, shape):
    """Packed projections with head sizes below 64 run fused in place (head
    stride D, K and V at column offsets C and 2C)."""
    bsz, n, heads, d = shape
    c = heads * d
    rng = np.random.default_rng(bsz + n + heads + d)
    qkv = rnd(rng, (bsz, n, 3 * c), 1.0, dtype)
    o = down(cu().dev_attention_packed(up(qkv, dtype), heads))
    o64 = dit.mha_f64(qkv[..., :c], qkv[..., c:2 * c], qkv[..., 2 * c:], heads)
    assert o.shape == (bsz, n, c)
    assert float(np.max(np.abs(o - o64))) <= attn_bound(qkv, dtype, n)


@pytest.mark.parametrize("dtype", ["bfloat16"])
def test_attention_packed_c5_shape_sampled_rows(dtype):
    """The packed C5 shape itself (17776 tokens, 30 heads of 64): 2100 work
    items of 256 query rows, 2048 run whole and the last 52 (head 29, rows
    4608 onwards) as key-range parts merged by the combine launch.  Sampled
    rows of whole and split items against fp64 over all 17776 keys."""
    n, heads = 17776, 30
    c = heads * 64
    rng = np.random.default_rng(17776)
    qkv = rnd(rng, (1, n, 3 * c), 1.0, dtype)
    o = down(cu().dev_attention_packed(up(qkv, dtype), heads))
    assert o.shape == (1, n, c)
    rows = np.array([0, 1, 255, 4607, 4608, 4609, 9000, 12345, 17520, 17775])
    for h in (0, 17, 28, 29):
        q = qkv[:, rows, h * 64:(h + 1) * 64]
        k = qkv[:, :, c + h * 64:c + (h + 1) * 64]
        v = qkv[:, :, 2 * c + h * 64:2 * c + (h + 1) * 64]
        o64 = ref.sdpa_f64(q, k, v, 0.125)
        err = float(np.max(np.abs(o[:, rows, h * 64:(h + 1) * 64] - o64)))
        assert err <= attn_bound(v, dtype, n), (h, err)


@pytest.mark.parametrize("sk", [1, 5, 63, 65, 100, 127, 200, 1000])
def test_fused_attention_ragged_keys(sk):
    """Key counts that are not multiples of the 64-key block: the tail is
    masked, and keys past Sk never contribute."""
    rng = np.random.default_rng(sk)
    q = rnd(rng, (2, 90, 64), 1.0, "bfloat16")
    k = rnd(rng, (2, sk, 64), 1.0, "bfloat16")
    v = rnd(rng, (2, sk, 64), 1.0, "bfloat16")
    g = cu()
    o = down(g.dev_scaled_dot_product_attention(up(q, "bfloat16"), up(k, "bfloat16"), up(v, "bfloat16"), 0.125))
    o64 = ref.sdpa_f64(q, k, v, 0.125)
    assert float(np.max(np.abs(o - o64))) <= attn_bound(v, "bfloat16", sk)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(2, 70, 33, 2, 64), (1, 40, 77, 4, 32), (2, 20, 9, 3, 40)],
                         ids=lambda s: "x".join(map(str, s)))
def test_multihead_attention(dtype, shape):
    """q (B, N, C), k and v (B, S, C): fused for 16-bit head sizes that are
    multiples of 8 up to 64 (64, 32, 40 here), the strided GEMM + softmax
    path for fp32."""
    bsz, n, s, heads, d = shape
    c = heads * d
    rng = np.random.default_rng(n * s + heads)
    q, k, v = (rnd(rng, (bsz, ln, c), 1.0, dtype) for ln in (n, s, s))
    o = down(cu().dev_multihead_attention(up(q, dtype), up(k, dtype), up(v, dtype), heads))
    o64 = dit.mha_f64(q, k, v, heads)
    bound = attn_bound(v, dtype, s)
    if dtype != "float32" and not (d % 8 == 0 and d <= 64):  # the unfused path rounds the scores too
        smax = float(np.max(np.abs(q.astype(np.float64)))) * float(np.max(np.abs(k.astype(np.float64)))) * d
        bound += 2 * {"float16": 2.0 ** -11, "bfloat16": 2.0 ** -8}[dtype] * smax / np.sqrt(d) * \
            float(np.max(np.abs(v)))
    assert float(np.max(np.abs(o - o64))) <= bound


def test_nonpositive_scale_takes_the_unfused_path():
    rng = np.random.default_rng(3)
    q, k, v = (rnd(rng, (1, 50, 64), 1.0, "float16") for _ in range(3))
    g = cu()
    for scale in (-0.125, 0.0):
        o = down(g.dev_scaled_dot_product_attention(up(q, "float16"), up(k, "float16"), up(v, "float16"), scale))
        o64 = ref.sdpa_f64(q, k, v, scale)
        assert np.all(np.isfinite(o))
        assert float(np.max(np.abs(o - o64))) <= 0.05
    so = _lib()
    P, I64 = ctypes.c_void_p, ctypes.c_int64
    x = up(np.zeros((64, 64), np.float32), "float16")
    p = P(x.data_ptr)
    rc = so.sf_attention(p, I64(64), I64(0), p, I64(64), I64(0), p, I64(64), I64(0), p, I64(64), I64(0),
                         I64(1), I64(64), I64(64), I64(64), ctypes.c_float(-1.0), 1, None)
    assert rc == -3 and b"scale" in so.sf_last_error()


def test_attention_heads_abi_overlap_check():
    so = _lib()
    P, I64 = ctypes.c_void_p, ctypes.c_int64
    x = up(np.zeros((4, 64, 256), np.float32), "bfloat16")
    p = P(x.data_ptr)

    def call(ldo, so_b, so_h, heads=4, batch=1):
        return so.sf_attention_heads(p, I64(256), I64(0), I64(64), p, I64(256), I64(0), I64(64), p, I64(256),
                                     I64(0), I64(64), p, I64(ldo), I64(so_b), I64(so_h), I64(batch),
                                     I64(heads), I64(16), I64(16), I64(64), ctypes.c_float(0.125), 2, None)
    assert call(256, 0, 32) == -2          # heads 32 apart overlap within a row
    assert call(128, 0, 64) == -2          # 4 heads of 64 do not fit a row of 128
    assert call(256, 100, 64, batch=2) == -2   # batch entries overlap
    cu().device_synchronize()


# ------------------------------------------------------------------ the whole block

def _block_params(rng, c, cd, ctx_dim, dtype):
    p = {}

    def lin(name, i, o, bias=True):
        k = 1.0 / np.sqrt(i)
        p[name + ".weight"] = quantize(rng.uniform(-k, k, (o, i)).astype(np.float32), dtype)
        if bias:
            p[name + ".bias"] = quantize(rng.uniform(-k, k, (o,)).astype(np.float32), dtype)

    for nm in ("norm1", "norm2", "norm3"):
        p[nm + ".norm.weight"] = quantize((1 + 0.1 * rng.standard_normal(c)).astype(np.float32), dtype)
        p[nm + ".norm.bias"] = quantize((0.1 * rng.standard_normal(c)).astype(np.float32), dtype)
        lin(nm + ".linear", cd, 2 * c)
    lin("to_qkv", c, 3 * c, bias=False)
    lin("self_out", c, c)
    if ctx_dim:
        lin("cross_q", c, c, bias=False)
        lin("cross_k", ctx_dim, c, bias=False)
        lin("cross_v", ctx_dim, c, bias=False)
        lin("cross_out", c, c)
    lin("ff.0", c, 4 * c)
    lin("ff.3", 4 * c, c)
    return p


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("cross", [False, True], ids=["self", "cross"])
def test_dit_block_matches_oracle(dtype, cross):
    import scaffolding_amd as sf
    from scaffolding_amd.diffusion import DiTBlock
    rng = np.random.default_rng(590 + cross)
    c, heads, cd, ctx_dim, n, s = 128, 2, 64, 96, 200, 33
    p = _block_params(rng, c, cd, ctx_dim if cross else 0, dtype)
    x = rnd(rng, (1, n, c), 1.0, dtype)
    cond = rnd(rng, (1, cd), 1.0, dtype)
    ctx = rnd(rng, (1, s, ctx_dim), 1.0, dtype) if cross else None
    blk = DiTBlock(c, heads, cd, ctx_dim if cross else 0, dtype=dtype)
    blk.load_state_dict(p)
    # loading kept no host copy and rounded on the device: the stored bits
    # equal the oracle's quantizer
    for name, prm in blk.state_dict().items():
        assert prm._data is None
        np.testing.assert_array_equal(prm.numpy(), p[name], err_msg=name)
    tx = sf.Tensor(x, dtype=dtype, device="cuda")
    tc = sf.Tensor(cond, dtype=dtype, device="cuda")
    tctx = sf.Tensor(ctx, dtype=dtype, device="cuda") if cross else None
    y = blk(tx, tc, tctx).numpy().astype(np.float64)
    assert y.shape == (1, n, c)
    if dtype == "float32":
        # the reference's own fp32 CPU path (diffusion/models.py:538-590)
        y_ref = dit.dit_block(x, cond, p, heads, context=ctx)
        assert normwise_err(y, y_ref) <= 1e-4
    else:
        ym = dit.dit_block_mirror(x, cond, p, heads, dtype, context=ctx)
        eps = out_half_ulp_rel(dtype)
        scale = float(np.max(np.abs(ym)))
        # a few output ulps: each launch rounds once, and rounding flips in
        # one launch's output move later launches by about an ulp of theirs
        assert float(np.max(np.abs(y - ym))) <= 16 * eps * scale, float(np.max(np.abs(y - ym)))
        assert normwise_err(y, ym) <= 4 * eps


def test_dit_block_state_dict_roundtrip_and_keys():
    from scaffolding_amd.diffusion import DiTBlock
    blk = DiTBlock(64, 1, 32, context_dim=16, dtype="bfloat16")
    keys = set(blk.state_dict())
    want = {"norm1.norm.weight", "norm1.norm.bias", "norm1.linear.weight", "norm1.linear.bias",
            "to_qkv.weight", "self_out.weight", "self_out.bias", "norm2.norm.weight", "norm2.norm.bias",
            "norm2.linear.weight", "norm2.linear.bias", "cross_q.weight", "cross_k.weight", "cross_v.weight",
            "cross_out.weight", "cross_out.bias", "norm3.norm.weight", "norm3.norm.bias", "norm3.linear.weight",
            "norm3.linear.bias", "ff.0.weight", "ff.0.bias", "ff.3.weight", "ff.3.bias"}
    assert keys == want
    other = DiTBlock(64, 1, 32, context_dim=16, dtype="bfloat16")
    w_before = other.to_qkv.weight
    other.load_state_dict({**blk.state_dict(), "unknown.key": np.zeros(3)})
    assert other.to_qkv.weight is w_before          # updated in place
    for k, v in blk.state_dict().items():
        assert np.array_equal(other.state_dict()[k].numpy(), v.numpy()), k


def test_multihead_fallback_head_groups_match():
    """The unfused path launches heads in groups that bound its score
    memory; one head per group and all heads at once give the same bits."""
    g = cu()
    rng = np.random.default_rng(44)
    q, k, v = (rnd(rng, (2, 30, 5 * 40), 1.0, "bfloat16") for _ in range(3))
    gq, gk, gv = up(q, "bfloat16"), up(k, "bfloat16"), up(v, "bfloat16")
    whole = down(g.dev_multihead_attention(gq, gk, gv, 5))
    saved = g._MHA_SCORES_BYTES
    try:
        g._MHA_SCORES_BYTES = 1
        one_by_one = down(g.dev_multihead_attention(gq, gk, gv, 5))
        g._MHA_SCORES_BYTES = 2 * 30 * 30 * 2
        pairs = down(g.dev_multihead_attention(gq, gk, gv, 5))
    finally:
        g._MHA_SCORES_BYTES = saved
    assert np.array_equal(whole, one_by_one) and np.array_equal(whole, pairs)
    o64 = dit.mha_f64(q, k, v, 5)
    assert float(np.max(np.abs(whole - o64))) <= 0.05


def test_split_workspace_two_threads_two_streams():
    """Split-tail GEMMs from two host threads on two streams share the
    per-device workspace: its lock spans each launch, so every result equals
    the single-threaded one bit for bit and the counters stay consistent."""
    import threading
    so = _lib()
    g = cu()
    P, I64 = ctypes.c_void_p, ctypes.c_int64
    rng = np.random.default_rng(3)
    m, n, k = 4352, 4096, 4096
    plan = g.gemm_plan(1, m, n, k, 1, 4096, k, 0, 8192, k, 0, n, m * n, "bfloat16")
    assert "split-tail" in plan, plan
    xs = [up(rnd(rng, (m, k), 1.0, "bfloat16"), "bfloat16") for _ in range(2)]
    w = up(rnd(rng, (n, k), 0.05, "bfloat16"), "bfloat16")
    outs = [g.empty((m, n), g.BFLOAT16) for _ in range(2)]
    g.device_synchronize()  # the uploads' casts ran on the default stream
    streams = []
    for _ in range(2):
        sp = ctypes.c_void_p()
        assert so.sf_stream_create(ctypes.byref(sp)) == 0
        streams.append(sp)

    def gemm(i, stream):
        return so.sf_gemm(0, 1, I64(m), I64(n), I64(k), I64(1), P(xs[i].data_ptr), I64(k), I64(0),
                          P(w.data_ptr), I64(k), I64(0), P(outs[i].data_ptr), I64(n), I64(0), 2, 2,
                          ctypes.c_float(1.0), None, 0, stream)
    want = []
    for i in range(2):
        assert gemm(i, streams[i]) == 0
        assert so.sf_stream_synchronize(streams[i]) == 0
        want.append(g.gputensor_bits_to_numpy(outs[i]).copy())
    errors = []

    def worker(i):
        for _ in range(40):
            rc = gemm(i, streams[i])
            if rc != 0:
                errors.append(rc)
                return
        so.sf_stream_synchronize(streams[i])

    ts = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors
    for i in range(2):
        assert np.array_equal(g.gputensor_bits_to_numpy(outs[i]), want[i])
    # and a later call is still right (the counters were left at zero)
    assert gemm(0, streams[0]) == 0 and so.sf_stream_synchronize(streams[0]) == 0
    assert np.array_equal(g.gputensor_bits_to_numpy(outs[0]), want[0])
    for sp in streams:
        so.sf_stream_destroy(sp)
