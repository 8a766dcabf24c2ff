"""Pins the oracle (CPU, no GPU) before anything is checked against it.

Each oracle function meets at least one check that a plausible mistake (a
dropped term, a wrong sign or index, a transposed operand) fails:
IEEE known answers for the quantizers, brute-force fsum fixtures for the
GEMM / linear restatements, closed-form identities for the activations,
invariants and a known answer for softmax / SDPA, the tolerance formulas
of BASELINE.json's north_star evaluated at tabulated sizes and the work
counts, and SHA-256 fingerprints for
the seeded config generators."""
from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest

from oracle import configs as cfg
from oracle import cpu_path as ref
from oracle.quant import bf16_bits, bf16_to_f32, quantize, round_bf16, round_f16

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _f32(bits):
    return np.array(bits, dtype=np.uint32).view(np.float32)


# ------------------------------------------------------------ quantizers

def test_bf16_known_answers():
    cases = {
        0x3F800000: 0x3F80,  # 1.0
        0x3F808000: 0x3F80,  # 1 + 2^-8: tie, even (down)
        0x3F818000: 0x3F82,  # 1 + 3*2^-8: tie, odd -> up
        0x3F80C000: 0x3F81,  # 1 + 3*2^-9 -> 1 + 2^-7
        0x3F807FFF: 0x3F80,  # just below the tie
        0x80000000: 0x8000,  # -0
        0x7F7FFFFF: 0x7F80,  # max finite rounds up to +inf
        0xFF7FFFFF: 0xFF80,
        0x7F7F7FFF: 0x7F7F,  # largest that stays finite
        0x7F800000: 0x7F80,  # +inf
        0xFF800000: 0xFF80,  # -inf
        0x00000001: 0x0000,  # smallest subnormal -> +0
        0x807FFFFF: 0x8080,  # largest negative subnormal -> -min normal
        0x00408000: 0x0040,  # subnormal tie, even
        0x00418000: 0x0042,  # subnormal tie, odd -> up
    }
    got = bf16_bits(_f32(list(cases)))
    assert [int(g) for g in got] == list(cases.values())
    nan = bf16_bits(_f32([0x7FC00000, 0xFFC00001, 0x7F800001]))
    assert np.all(np.isnan(bf16_to_f32(nan)))
    assert int(nan[1]) & 0x8000  # sign kept


def test_bf16_roundtrip_and_monotone():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(100000).astype(np.float32) * 1000
    r = round_bf16(x)
    assert np.array_equal(round_bf16(r), r)                     # idempotent
    assert np.all(np.abs(r - x) <= np.abs(x) * 2.0 ** -8)       # half-ulp bound
    xs = np.sort(x)
    assert np.all(np.diff(round_bf16(xs)) >= 0)                 # monotone
    # widening is exact: the upper 16 bits carry the value
    assert np.array_equal(bf16_to_f32(bf16_bits(r)).view(np.uint32) & 0xFFFF, np.zeros(r.size, np.uint32))


def test_f16_known_answers():
    x = np.array([1.0, 2049.0, 2051.0, 65504.0, 65519.0, 65520.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26],
                 np.float32)
    with np.errstate(over="ignore"):
        got = round_f16(x)
    want = [1.0, 2048.0, 2052.0, 65504.0, 65504.0, np.inf, 2.0 ** -24, 0.0, 2.0 ** -24]
    assert list(got) == want
    assert quantize(x[:3], "float32") is not None


# ------------------------------------------------------------ GEMM / linear

def test_matmul_against_bruteforce_fixtures():
    fx = np.load(os.path.join(GOLDEN, "tiny_gemm.npz"))
    keys = sorted(k[:-2] for k in fx.files if k.endswith("_c"))
    assert len(keys) == 18
    for key in keys:
        a, b, c = fx[key + "_a"], fx[key + "_b"], fx[key + "_c"]
        got = ref.matmul_f64(a, b)
        np.testing.assert_allclose(got, c, rtol=1e-13, atol=1e-13, err_msg=key)
        # the NT restatement on B^T gives the same product
        np.testing.assert_allclose(ref.matmul_nt(a.astype(np.float64), np.ascontiguousarray(b.T, np.float64)), c,
                                   rtol=1e-13, atol=1e-13)
        # fp32 CPU path within fp32 accumulation error of the exact value
        k = a.shape[1]
        bound = k * 2.0 ** -23 * (np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))) + 1e-30
        assert np.all(np.abs(ref.matmul(a, b) - c) <= bound)


def test_bruteforce_matches_triple_loop_definition():
    a = [[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]]
    b = [[7.0, 8.0], [9.0, 10.0], [11.0, 12.0]]
    assert ref.matmul_bruteforce(a, b) == [[58.0, 64.0], [139.0, 154.0]]


def test_planted_mistakes_are_caught():
    """A transposed operand, a dropped bias or a sign flip in the oracle
    would not reproduce the fixtures."""
    fx = np.load(os.path.join(GOLDEN, "tiny_gemm.npz"))
    a, b, c = fx["float32_7x6x24_a"], fx["float32_7x6x24_b"], fx["float32_7x6x24_c"]
    with pytest.raises(ValueError):
        np.matmul(a, b.T)  # transposed B does not even conform here
    sq_a, sq_b, sq_c = fx["float32_4x3x2_a"], fx["float32_4x3x2_b"], fx["float32_4x3x2_c"]
    assert not np.allclose(-ref.matmul_f64(sq_a, sq_b), sq_c)
    lx = np.load(os.path.join(GOLDEN, "tiny_linear.npz"))
    x, w, bias, want = lx["float32_3x5x7_x"], lx["float32_3x5x7_w"], lx["float32_3x5x7_b"], lx["float32_3x5x7_bias"]
    assert not np.allclose(ref.linear_f64(x, w, None), want)       # dropped bias
    assert np.allclose(ref.linear_f64(x, w, bias), want, rtol=1e-13, atol=1e-13)
    assert c.shape == (7, 6)


@pytest.mark.parametrize("dt", ["float32", "float16", "bfloat16"])
def test_linear_epilogues_against_fixtures(dt):
    fx = np.load(os.path.join(GOLDEN, "tiny_linear.npz"))
    for shape in ("3x5x7", "2x4x16"):
        key = "%s_%s" % (dt, shape)
        x, w, b = fx[key + "_x"], fx[key + "_w"], fx[key + "_b"]
        np.testing.assert_allclose(ref.linear_f64(x, w, b), fx[key + "_bias"], rtol=1e-13, atol=1e-13)
        np.testing.assert_allclose(ref.linear_f64(x, w, b, "silu"), fx[key + "_silu"], rtol=1e-12, atol=1e-13)
        np.testing.assert_allclose(ref.linear_f64(x, w, b, "gelu"), fx[key + "_gelu"], rtol=1e-12, atol=1e-13)
        # the fp32 CPU restatement (x @ W.T + b, then silu) within fp32 error
        y32 = ref.silu(ref.linear(x, w, b))
        assert np.allclose(y32, fx[key + "_silu"], rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------ backward

def test_linear_backward_against_fixtures():
    """LinearBackward (reference autograd.py:793-822): the fp64 closed form
    equals the math.fsum fixtures, and the fp32 NumPy restatement is within
    fp32 accumulation error of them."""
    fx = np.load(os.path.join(GOLDEN, "tiny_backward.npz"))
    keys = sorted(k[:-2] for k in fx.files if k.endswith("_g"))
    assert len(keys) == 12
    for key in keys:
        g, x, w = fx[key + "_g"], fx[key + "_x"], fx[key + "_w"]
        dx, dw, db = ref.linear_backward_f64(g, x, w)
        np.testing.assert_allclose(dx, fx[key + "_dx"], rtol=1e-13, atol=1e-13, err_msg=key)
        np.testing.assert_allclose(dw, fx[key + "_dw"], rtol=1e-13, atol=1e-13, err_msg=key)
        np.testing.assert_allclose(db, fx[key + "_db"], rtol=1e-13, atol=1e-13, err_msg=key)
        np.testing.assert_allclose(ref.matmul_tn(g.astype(np.float64), x.astype(np.float64)), fx[key + "_dw"],
                                   rtol=1e-13, atol=1e-13)
        np.testing.assert_allclose(ref.sum_dim(g.astype(np.float64), 0), fx[key + "_db"], rtol=1e-13, atol=1e-13)
        gi, gw, gb = ref.linear_backward(g, x, w)
        m = g.shape[0]
        ag, ax, aw = (np.abs(v.astype(np.float64)) for v in (g, x, w))
        assert np.all(np.abs(gi - fx[key + "_dx"]) <= g.shape[1] * 2.0 ** -23 * (ag @ aw) + 1e-30)
        assert np.all(np.abs(gw - fx[key + "_dw"]) <= m * 2.0 ** -23 * (ag.T @ ax) + 1e-30)
        assert np.all(np.abs(gb - fx[key + "_db"]) <= m * 2.0 ** -23 * ag.sum(axis=0) + 1e-30)
        assert ref.linear_backward(g, x, w, has_bias=False)[1].shape == w.shape


def test_backward_planted_mistakes_are_caught():
    """A sign flip, a misaligned row pairing or a sum over the wrong axis
    would not reproduce the fixtures."""
    fx = np.load(os.path.join(GOLDEN, "tiny_backward.npz"))
    key = "float32_9x6x16"
    g, x, w = (fx[key + s].astype(np.float64) for s in ("_g", "_x", "_w"))
    assert not np.allclose(-(g.T @ x), fx[key + "_dw"])
    assert not np.allclose(g.T @ np.roll(x, 1, axis=0), fx[key + "_dw"])
    assert g.sum(axis=1).shape != fx[key + "_db"].shape
    with pytest.raises(ValueError):
        np.matmul(g, w.T)  # grad_input with W transposed does not conform


def test_sum_dim_shapes_follow_reference():
    """dev_sum_dim's output shapes (reference _cuda_ops.pyx:1710-1741)."""
    x = np.arange(24, dtype=np.float64).reshape(2, 3, 4)
    assert ref.sum_dim(x, 1).shape == (2, 4)
    assert ref.sum_dim(x, 1, keepdim=True).shape == (2, 1, 4)
    assert ref.sum_dim(x, -1).shape == (2, 3)
    assert ref.sum_dim(np.arange(5.0), 0).shape == ()  # the device op returns (1,)
    np.testing.assert_array_equal(ref.sum_dim(x, 0), x[0] + x[1])


# ------------------------------------------------------------ activations

def test_silu_closed_forms():
    x = np.linspace(-20, 20, 4001)
    np.testing.assert_allclose(ref.silu(x), 0.5 * x * (1.0 + np.tanh(0.5 * x)), rtol=1e-12, atol=1e-15)
    assert ref.silu(np.array([0.0]))[0] == 0.0
    big = np.array([50.0, 80.0])
    np.testing.assert_allclose(ref.silu(big), big, rtol=1e-15)
    assert np.all(np.abs(ref.silu(np.array([-50.0, -80.0]))) < 1e-19)
    np.testing.assert_allclose(ref.act_f64(x, "silu"), ref.silu(x), rtol=1e-12, atol=1e-15)


def test_gelu_closed_forms():
    x = np.linspace(-12, 12, 2401)
    g = ref.gelu_tanh(x)
    np.testing.assert_allclose(g - ref.gelu_tanh(-x), x, rtol=1e-12, atol=1e-12)   # tanh is odd
    assert ref.gelu_tanh(np.array([0.0]))[0] == 0.0
    np.testing.assert_allclose(ref.gelu_tanh(np.array([30.0])), [30.0], rtol=1e-15)
    # the tanh form approximates the exact erf GELU to within 5e-4 everywhere
    erf_gelu = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x])
    assert np.max(np.abs(g - erf_gelu)) < 5e-4
    # the sigmoid form used by the kernels is the same function
    u = math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)
    np.testing.assert_allclose(x / (1 + np.exp(-2 * u)), g, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(ref.act_f64(x, "gelu"), g, rtol=1e-12, atol=1e-15)


# ------------------------------------------------------------ softmax / SDPA

def test_softmax_invariants_and_known_answer():
    p = ref.softmax(np.array([[0.0, math.log(2.0)]]))
    np.testing.assert_allclose(p, [[1 / 3, 2 / 3]], rtol=1e-15)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((9, 37)) * 5
    p = ref.softmax(x.copy())
    np.testing.assert_allclose(p.sum(axis=-1), 1.0, rtol=1e-14)
    np.testing.assert_allclose(ref.softmax(x + 100.0), p, rtol=1e-12)
    np.testing.assert_allclose(ref.softmax(np.full((2, 5), 3.0)), np.full((2, 5), 0.2))
    np.testing.assert_allclose(ref.softmax_f64(x, 0.5), ref.softmax(0.5 * x), rtol=1e-12)


def test_sdpa_known_answers():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((2, 6, 4))
    v = rng.standard_normal((2, 6, 4))
    k0 = np.zeros((2, 6, 4))
    # equal scores: every query averages the values
    np.testing.assert_allclose(ref.sdpa(q, k0, v), np.broadcast_to(v.mean(axis=1, keepdims=True), v.shape),
                               rtol=1e-12, atol=1e-12)
    # V = identity: the output is the probability matrix itself
    k = rng.standard_normal((1, 4, 4))
    eye = np.eye(4)[None]
    p = ref.softmax_f64(q[:1, :4] @ np.swapaxes(k, -2, -1), 0.5)
    np.testing.assert_allclose(ref.sdpa_f64(q[:1, :4], k, eye, 0.5), p, rtol=1e-12)
    np.testing.assert_allclose(ref.sdpa(q, k0 + q, v, 0.7), ref.sdpa_f64(q, q, v, 0.7), rtol=1e-10, atol=1e-12)


MASK_CASES = ["qk", "b1qk", "bh1k", "1k"]


@pytest.mark.parametrize("name", MASK_CASES)
def test_sdpa_mask_against_fsum_fixture(name):
    """The additive mask (reference nn/functional.py:339-341) against the
    fsum fixture, over four broadcast shapes with -inf entries; in fp32
    (the reference's own restatement) and fp64."""
    z = np.load(os.path.join(GOLDEN, "tiny_mask.npz"))
    key = "mask_" + name
    q, k, v, mask, o = (z[key + s] for s in ("_q", "_k", "_v", "_mask", "_o"))
    scale = 1.0 / math.sqrt(q.shape[-1])
    np.testing.assert_allclose(ref.sdpa_f64(q, k, v, scale, mask), o, rtol=1e-12, atol=1e-13)
    got = ref.sdpa(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), None, mask.astype(np.float32))
    np.testing.assert_allclose(got, o, rtol=2e-5, atol=2e-6)


def test_sdpa_mask_planted_mistakes_fail():
    """Plausible mistakes in applying the mask are caught by the fixture:
    the mask ignored, added before the scale instead of after it, or only
    its -inf entries applied (finite values dropped)."""
    z = np.load(os.path.join(GOLDEN, "tiny_mask.npz"))
    scale = 1.0 / math.sqrt(8)
    for name in MASK_CASES:
        key = "mask_" + name
        q, k, v, mask, o = (z[key + s] for s in ("_q", "_k", "_v", "_mask", "_o"))
        s = q @ np.swapaxes(k, -2, -1)
        wrong = [ref.sdpa_f64(q, k, v, scale), ref.softmax_f64(s + mask, scale) @ v,
                 ref.sdpa_f64(q, k, v, scale, np.where(np.isfinite(mask), 0.0, mask))]
        for w in wrong:
            assert not np.allclose(np.nan_to_num(w), o, rtol=1e-6, atol=1e-6), name


# ------------------------------------------------------------ tolerances, counts, generators

def test_tolerances_match_baseline_table():
    assert cfg.tol_16(4096) == pytest.approx(4.0e-2)
    assert cfg.tol_16(64) == pytest.approx(5.0e-3)
    assert cfg.tol_16(1920) == pytest.approx(2.739e-2, rel=1e-3)
    assert cfg.tol_16(7680) == pytest.approx(5.477e-2, rel=1e-3)
    assert cfg.tol_fp32(512) == pytest.approx(2.263e-4, rel=1e-3)
    assert cfg.tol_fp32(1024) == pytest.approx(3.20e-4, rel=1e-2)
    assert cfg.tol_fp32(4096) == pytest.approx(6.40e-4, rel=1e-2)


def test_work_counts_match_baseline_table():
    assert cfg.gemm_flops(64, 512, 512) == pytest.approx(33.55e6, rel=1e-3)
    assert cfg.gemm_bytes(1, 11008, 4096, 2, 2, bias=True) / 1e6 == pytest.approx(90.23, rel=1e-3)
    assert cfg.gemm_bytes(16, 11008, 4096, 2, 2, bias=True) / 1e6 == pytest.approx(90.68, rel=1e-3)
    assert cfg.gemm_flops(4096, 11008, 4096) / 1e9 == pytest.approx(369.4, rel=1e-3)
    assert cfg.gemm_flops(4096, 4096, 64, 60) / 1e9 == pytest.approx(128.8, rel=1e-3)
    assert cfg.C5_TOKENS == 17776
    assert cfg.gemm_flops(17776, 5760, 1920) / 1e9 == pytest.approx(393.2, rel=1e-3)


def test_config_generators_are_pinned():
    with open(os.path.join(GOLDEN, "config_inputs.json")) as f:
        want = json.load(f)
    import hashlib

    def dig(a):
        a = np.ascontiguousarray(a, dtype=np.float32)
        return list(a.shape), hashlib.sha256(a.tobytes()).hexdigest()

    c1 = cfg.c1_linear()
    for name, arr in (("x", c1.x), ("w", c1.w), ("b", c1.b)):
        assert dig(arr) == (want["C1"][name]["shape"], want["C1"][name]["sha256"]), name
    a, b = cfg.c2_matmul(1024)
    assert dig(a)[1] == want["C2_1024"]["a"]["sha256"] and dig(b)[1] == want["C2_1024"]["b"]["sha256"]
    c3 = cfg.c3_linear(16)
    assert dig(c3.w)[1] == want["C3_M16"]["w"]["sha256"]
    q, k, v, _ = cfg.c4_attention()
    assert dig(v)[1] == want["C4"]["v"]["sha256"]
    # quantized to the config dtype (bf16 values are exactly representable)
    assert np.array_equal(round_bf16(c3.x), c3.x)
    assert np.array_equal(round_f16(q), q)
