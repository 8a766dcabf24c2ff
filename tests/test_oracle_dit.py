"""Pins the DiT-block oracle (oracle/dit.py) on the CPU: the float64 closed
forms and the fp32 restatement of the reference against the pure-Python
math.fsum fixtures of tests/golden/make_golden.py (tiny_norm.npz,
tiny_dit.npz), against invariants the mathematics fixes, and against
planted mistakes that must fail the fixtures."""
from __future__ import annotations

import math
import os

import numpy as np
import pytest

from oracle import cpu_path as ref
from oracle import dit

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def norm_fx():
    return np.load(os.path.join(GOLDEN, "tiny_norm.npz"))


@pytest.fixture(scope="module")
def dit_fx():
    d = np.load(os.path.join(GOLDEN, "tiny_dit.npz"))
    p = {k[2:]: d[k] for k in d.files if k.startswith("p_")}
    return d, p


SHAPES = [(1, 1), (3, 5), (4, 16), (2, 37)]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "%dx%d" % s)
def test_layer_norm_matches_fsum_fixture(norm_fx, shape):
    key = "ln_%dx%d" % shape
    x, g, b = norm_fx[key + "_x"], norm_fx[key + "_g"], norm_fx[key + "_b"]
    ms, mt = norm_fx[key + "_ms"], norm_fx[key + "_mt"]
    np.testing.assert_allclose(dit.layer_norm_f64(x, g, b, 1e-5), norm_fx[key + "_y"], rtol=0, atol=1e-12)
    np.testing.assert_allclose(dit.layer_norm_f64(x, g, b, 1e-5, ms, mt), norm_fx[key + "_ymod"], rtol=0,
                               atol=1e-12)
    # the fp32 restatement of the reference (nn/layers.py:512-521)
    y32 = dit.layer_norm(x.astype(np.float32), g.astype(np.float32), b.astype(np.float32), 1e-5)
    np.testing.assert_allclose(y32, norm_fx[key + "_y"], rtol=0, atol=2e-5)


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "%dx%d" % s)
def test_rms_norm_matches_fsum_fixture(norm_fx, shape):
    key = "ln_%dx%d" % shape
    x, g = norm_fx[key + "_x"], norm_fx[key + "_g"]
    np.testing.assert_allclose(dit.rms_norm_f64(x, g, 1e-6), norm_fx["rms_%dx%d_y" % shape], rtol=0, atol=1e-12)
    y32 = dit.rms_norm(x.astype(np.float32), g.astype(np.float32), 1e-6)
    np.testing.assert_allclose(y32, norm_fx["rms_%dx%d_y" % shape], rtol=0, atol=2e-5)


def test_layer_norm_invariants():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((6, 300)) * 3 + 5
    y = dit.layer_norm_f64(x, eps=0.0)
    np.testing.assert_allclose(y.mean(axis=-1), 0, atol=1e-12)
    np.testing.assert_allclose((y ** 2).mean(axis=-1), 1, atol=1e-12)
    # invariant to positive scaling and shifting of a row (eps = 0)
    np.testing.assert_allclose(dit.layer_norm_f64(2.5 * x - 7, eps=0.0), y, atol=1e-11)
    # zero modulation is the plain norm; scale -1 zeroes it, leaving the shift
    z = np.zeros_like(x)
    np.testing.assert_allclose(dit.layer_norm_f64(x, eps=1e-5, mod_scale=z, mod_shift=z),
                               dit.layer_norm_f64(x, eps=1e-5), atol=0)
    np.testing.assert_allclose(dit.layer_norm_f64(x, eps=1e-5, mod_scale=z - 1, mod_shift=z + 0.25), 0.25,
                               atol=1e-15)
    # RMS norm of a row with zero mean equals layer norm (eps = 0)
    xc = x - x.mean(axis=-1, keepdims=True)
    np.testing.assert_allclose(dit.rms_norm_f64(xc, eps=0.0), dit.layer_norm_f64(xc, eps=0.0), atol=1e-12)


@pytest.mark.parametrize("shape", [(1, 1, 4), (3, 5, 8), (4, 67, 8)], ids=lambda s: "x".join(map(str, s)))
def test_attention_matches_fsum_fixture(norm_fx, shape):
    key = "attn_%dx%dx%d" % shape
    q, k, v, o = (norm_fx[key + s] for s in ("_q", "_k", "_v", "_o"))
    d = shape[2]
    np.testing.assert_allclose(ref.sdpa_f64(q, k, v, 1.0 / math.sqrt(d)), o, rtol=0, atol=1e-13)
    # one head through the packed-heads closed form
    np.testing.assert_allclose(dit.mha_f64(q[None], k[None], v[None], 1)[0], o, rtol=0, atol=1e-13)
    # the reference's fp32 _attn (with its + 1e-9 in the denominator)
    o32 = dit.dit_attn(*(a.astype(np.float32)[None, None] for a in (q, k, v)))[0, 0]
    np.testing.assert_allclose(o32, o, rtol=0, atol=1e-6)


@pytest.mark.parametrize("cross", [False, True], ids=["self", "cross"])
def test_dit_block_matches_fsum_fixture(dit_fx, cross):
    d, p = dit_fx
    ctx = d["context"] if cross else None
    want = d["y_cross"] if cross else d["y_self"]
    heads = int(d["heads"])
    y = dit.dit_block_mirror(d["x"], d["cond"], p, heads, None, context=ctx)
    np.testing.assert_allclose(y, want, rtol=0, atol=1e-12)
    p32 = {k: v.astype(np.float32) for k, v in p.items()}
    y32 = dit.dit_block(d["x"].astype(np.float32), d["cond"].astype(np.float32), p32, heads,
                        context=None if ctx is None else ctx.astype(np.float32))
    np.testing.assert_allclose(y32, want, rtol=0, atol=5e-5)


def _mirror_with(monkeypatch, d, p, **patch):
    for name, fn in patch.items():
        monkeypatch.setattr(dit, name, fn)
    return dit.dit_block_mirror(d["x"], d["cond"], p, int(d["heads"]), None, context=d["context"])


def test_planted_mistakes_fail_the_dit_fixture(dit_fx, monkeypatch):
    """Each plausible mistake moves the tiny block's output far beyond the
    1e-12 the closed form meets."""
    d, p = dit_fx
    want = d["y_cross"]
    orig_ln, orig_split, orig_merge = dit.layer_norm_f64, dit.split_heads, dit.merge_heads

    def no_plus_one(x, g=None, b=None, eps=1e-5, mod_scale=None, mod_shift=None):
        h = orig_ln(x, g, b, eps)
        return h * mod_scale + mod_shift if mod_scale is not None else h

    def split_hd(t, heads):  # heads taken as the inner factor of C
        b, n, c = t.shape
        return t.reshape(b, n, c // heads, heads).transpose(0, 3, 1, 2).copy()

    def merge_hd(t):
        b, h, n, dd = t.shape
        return t.transpose(0, 2, 3, 1).reshape(b, n, h * dd).copy()

    def no_gamma(x, g=None, b=None, eps=1e-5, mod_scale=None, mod_shift=None):
        return orig_ln(x, None, b, eps, mod_scale, mod_shift)

    for patch in (dict(layer_norm_f64=no_plus_one), dict(split_heads=split_hd, merge_heads=merge_hd),
                  dict(layer_norm_f64=no_gamma)):
        with monkeypatch.context() as m:
            y = _mirror_with(m, d, p, **patch)
        assert float(np.max(np.abs(y - want))) > 1e-3, patch
    assert dit.layer_norm_f64 is orig_ln and dit.split_heads is orig_split and dit.merge_heads is orig_merge
    # dropping the cross-attention block, or zeroing the block input the
    # residuals carry, fails too
    assert float(np.max(np.abs(d["y_self"] - want))) > 1e-3
    y_nores = dit.dit_block_mirror(d["x"] * 0, d["cond"], p, int(d["heads"]), None, context=d["context"])
    assert float(np.max(np.abs(y_nores - want))) > 1e-3


def test_mirror_rounds_at_launch_boundaries(dit_fx):
    """dtype rounding only moves the result by rounding-sized amounts, and
    every returned value is representable in the dtype."""
    from oracle.quant import quantize
    d, p = dit_fx
    heads = int(d["heads"])
    pq = {k: quantize(v.astype(np.float32), "bfloat16").astype(np.float64) for k, v in p.items()}
    xq = quantize(d["x"].astype(np.float32), "bfloat16").astype(np.float64)
    cq = quantize(d["cond"].astype(np.float32), "bfloat16").astype(np.float64)
    y16 = dit.dit_block_mirror(xq, cq, pq, heads, "bfloat16")
    y64 = dit.dit_block_mirror(xq, cq, pq, heads, None)
    assert np.array_equal(quantize(y16.astype(np.float32), "bfloat16"), y16.astype(np.float32))
    assert 0 < float(np.max(np.abs(y16 - y64))) < 0.1
