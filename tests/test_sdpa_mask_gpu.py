"""scaled_dot_product_attention with an additive attn_mask on the device
(sf_softmax_rows_masked inside the three-launch path) against the oracle's
restatement of the reference's masked branch (nn/functional.py:339-341:
scores *= scale; scores += mask, NumPy broadcasting; oracle.cpu_path.sdpa
and its fp64 twin sdpa_f64, both pinned by tests/golden/tiny_mask.npz),
and the fused path's fallback when sf_attention declines a call."""
from __future__ import annotations

import ctypes
import math
import os

import numpy as np
import pytest

from helpers import cu, rnd, up
from oracle import cpu_path as ref
from oracle.configs import tol_16, tol_fp32

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
EPS = {"float32": 2.0 ** -24, "float16": 2.0 ** -11, "bfloat16": 2.0 ** -8}


def down(gt):
    return cu().gputensor_to_numpy(gt).astype(np.float32)


def bound(q, k, v, scale, dtype):
    """The three-launch path's bound: BASELINE's GEMM tolerance at K = Sk
    (fp32: relative to max|o|), P and the output rounded to the dtype
    (eps * max|v| each), and the scaled scores rounded before the mask is
    added (|d p| <= p * 2 eps |s|: 2 eps max|s| max|v|)."""
    eps = EPS[dtype]
    vmax = float(np.max(np.abs(v)))
    smax = float(np.max(np.abs(scale * (q.astype(np.float64) @ np.swapaxes(k.astype(np.float64), -1, -2)))))
    base = tol_fp32(k.shape[-2]) * vmax if dtype == "float32" else tol_16(k.shape[-2])
    return base + 2 * eps * vmax + 2 * eps * smax * vmax


def make_mask(rng, shape, dtype, ninf_frac=0.15):
    m = rng.uniform(-4.0, 4.0, shape).astype(np.float32)
    if ninf_frac > 0:
        flat = m.reshape(-1)
        flat[rng.random(flat.size) < ninf_frac] = -np.inf
    if dtype != "float32":
        from oracle.quant import quantize
        m = quantize(m, dtype)
    return m


MASK_SHAPES = [(130, 200), (2, 1, 130, 200), (2, 3, 1, 200), (200,), (2, 3, 130, 200), (1, 3, 1, 1), (3, 130, 1)]


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("mshape", MASK_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_masked_sdpa_matches_fp64(dtype, mshape):
    """[2, 3, 130, 200] scores (Sk a multiple of 8: one wave per row) with
    masks of seven broadcast shapes, -inf entries included; the mask in
    the scores' dtype."""
    rng = np.random.default_rng(len(mshape) * 100 + sum(mshape))
    q = rnd(rng, (2, 3, 130, 64), 1.0, dtype)
    k = rnd(rng, (2, 3, 200, 64), 1.0, dtype)
    v = rnd(rng, (2, 3, 200, 64), 1.0, dtype)
    mask = make_mask(rng, mshape, dtype, 0.15 if mshape[-1] > 1 else 0.0)
    full = np.broadcast_to(mask, (2, 3, 130, 200))
    assert np.all(np.isfinite(full).any(axis=-1))
    g = cu()
    gm = up(mask, dtype)
    o = down(g.dev_scaled_dot_product_attention(up(q, dtype), up(k, dtype), up(v, dtype), None, gm))
    scale = 1.0 / 8.0
    o64 = ref.sdpa_f64(q, k, v, scale, mask)
    assert o.shape == (2, 3, 130, 64) and np.all(np.isfinite(o))
    err = float(np.max(np.abs(o - o64)))
    assert err <= bound(q, k, v, scale, dtype), err
    if dtype == "float32":
        # the reference's own fp32 restatement of the masked branch
        o32 = ref.sdpa(q, k, v, scale, mask)
        assert float(np.max(np.abs(o - o32))) <= bound(q, k, v, scale, dtype)


@pytest.mark.parametrize("dtype,mdtype", [("bfloat16", "float32"), ("float16", "float32"), ("bfloat16", "float16")])
def test_masked_sdpa_mask_dtypes_and_ragged_keys(dtype, mdtype):
    """Sk = 203 (not a multiple of 8: one block per row), head size 40, a
    [Sq, Sk] mask in fp32 or in another 16-bit dtype (converted to fp32 on
    the device first)."""
    rng = np.random.default_rng(203)
    q = rnd(rng, (3, 70, 40), 1.0, dtype)
    k = rnd(rng, (3, 203, 40), 1.0, dtype)
    v = rnd(rng, (3, 203, 40), 1.0, dtype)
    mask = make_mask(rng, (70, 203), mdtype)
    g = cu()
    o = down(g.dev_scaled_dot_product_attention(up(q, dtype), up(k, dtype), up(v, dtype), 0.3, up(mask, mdtype)))
    o64 = ref.sdpa_f64(q, k, v, 0.3, mask)
    assert float(np.max(np.abs(o - o64))) <= bound(q, k, v, 0.3, dtype)


@pytest.mark.parametrize("name", ["qk", "b1qk", "bh1k", "1k"])
def test_masked_sdpa_golden_fixture(name):
    """The fsum fixture (tests/golden/tiny_mask.npz) through the device in
    fp32, through the Tensor API with a host-array mask."""
    import scaffolding_amd as sf
    from scaffolding_amd.nn import functional as F
    z = np.load(os.path.join(GOLDEN, "tiny_mask.npz"))
    key = "mask_" + name
    q, k, v, mask, o = (z[key + s].astype(np.float32) for s in ("_q", "_k", "_v", "_mask", "_o"))
    dev = sf.device("cuda:0")
    tq, tk, tv = (sf.Tensor(a, device=dev) for a in (q, k, v))
    got = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=mask).numpy()
    assert got.shape == o.shape
    np.testing.assert_allclose(got, o, rtol=0, atol=2e-5 * float(np.max(np.abs(v))) + 1e-6)
    # a device Tensor mask gives the same bits
    got2 = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=sf.Tensor(mask, device=dev)).numpy()
    assert np.array_equal(got, got2)


def test_masked_sdpa_refusals():
    """A mask that does not broadcast, or a dropout_p outside [0, 1), is
    refused before any launch; a fully masked row gives NaN, as the
    reference's NumPy does."""
    from scaffolding_amd.nn import functional as F
    import scaffolding_amd as sf
    g = cu()
    rng = np.random.default_rng(5)
    q = rnd(rng, (2, 16, 64), 1.0, "float32")
    gq = up(q, "float32")
    with pytest.raises(ValueError, match="broadcast"):
        g.dev_scaled_dot_product_attention(gq, gq, gq, None, up(np.zeros((3, 16, 16), np.float32), "float32"))
    dev = sf.device("cuda:0")
    tq = sf.Tensor(q, device=dev)
    with pytest.raises(ValueError, match="dropout_p"):
        F.scaled_dot_product_attention(tq, tq, tq, dropout_p=-0.1)
    mask = np.zeros((16, 16), np.float32)
    mask[3, :] = -np.inf
    o = down(g.dev_scaled_dot_product_attention(gq, gq, gq, None, up(mask, "float32")))
    with np.errstate(invalid="ignore"):
        o64 = ref.sdpa(q, q, q, None, mask)
    assert np.all(np.isnan(o[:, 3])) and np.all(np.isnan(o64[:, 3]))
    assert np.all(np.isfinite(np.delete(o, 3, axis=1)))


def test_sdpa_falls_back_when_the_fused_kernel_declines():
    """K and V of one batch entry at 2 GiB: sf_attention returns
    SF_ERR_UNSUPPORTED (its key offsets are 32-bit), and
    dev_scaled_dot_product_attention runs the three-launch path instead of
    raising.  K and V are zero except four key rows, so the fp64 answer is
    cheap on the host: 2^24 - 4 keys score 0, the four score about 12-16."""
    g = cu()
    lib = ctypes.CDLL(os.path.join(ROOT, "scaffolding_amd", "libsfgemm.so"))
    lib.sf_last_error.restype = ctypes.c_char_p
    dt = "float16"
    sq, sk, d = 8, 1 << 24, 64
    rng = np.random.default_rng(24)
    q = rnd(rng, (1, sq, d), 1.0, dt)
    special = np.array([0, 12345, sk // 2 + 3, sk - 1])
    # k_j = a_j q_0 / |q_0|^2 * 8: row 0 scores a_j (scale 1/8)
    a = np.array([12.0, 14.0, 16.0, 15.0])
    krows = quantizef16(a[:, None] * q[0, 0][None, :] * 8.0 / float(q[0, 0] @ q[0, 0]))
    vrows = rnd(rng, (4, d), 1.0, dt)
    print("sdpa fallback: 1 x %d x %d fp16 keys (2 GiB K and V)" % (sk, d), flush=True)
    gq = up(q, dt)
    gk = g.zeros((1, sk, d), np.float16)
    gv = g.zeros((1, sk, d), np.float16)
    gkr, gvr = up(krows, dt), up(vrows, dt)
    for i, j in enumerate(special):
        for dst, src in ((gk, gkr), (gv, gvr)):
            assert lib.sf_memcpy_d2d(ctypes.c_void_p(dst.data_ptr + int(j) * d * 2),
                                     ctypes.c_void_p(src.data_ptr + i * d * 2), ctypes.c_size_t(d * 2), None) == 0
    go = g.zeros((1, sq, d), np.float16)
    I64 = ctypes.c_int64
    rc = lib.sf_attention(ctypes.c_void_p(gq.data_ptr), I64(d), I64(sq * d), ctypes.c_void_p(gk.data_ptr), I64(d),
                          I64(sk * d), ctypes.c_void_p(gv.data_ptr), I64(d), I64(sk * d),
                          ctypes.c_void_p(go.data_ptr), I64(d), I64(sq * d), I64(1), I64(sq), I64(sk), I64(d),
                          ctypes.c_float(0.125), 1, None)
    assert rc == -3 and b"2 GiB" in lib.sf_last_error(), rc
    o = down(g.dev_scaled_dot_product_attention(gq, gk, gv, 0.125))
    # fp64: scores s_j on the four rows, 0 on the other sk - 4
    s = 0.125 * (q[0].astype(np.float64) @ krows.astype(np.float64).T)  # [sq, 4]
    m = np.maximum(s.max(axis=1, keepdims=True), 0.0)
    e = np.exp(s - m)
    z = e.sum(axis=1, keepdims=True) + (sk - 4) * np.exp(-m)
    o64 = (e / z) @ vrows.astype(np.float64)
    assert np.all(np.isfinite(o))
    # scores of ~16 rounded to fp16 (half ulp 2^-7) move a weight by < 1 %
    err = float(np.max(np.abs(o[0] - o64)))
    assert err <= 2e-2 * float(np.max(np.abs(vrows))), err
    assert float(np.max(np.abs(o64[0]))) > 0.1  # row 0's answer is not the background's


def quantizef16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)
