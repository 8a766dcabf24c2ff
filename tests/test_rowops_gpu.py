"""Row / elementwise kernels on the GPU: dtype casts (bit-exact against the
oracle's RNE), softmax, SiLU, GELU-tanh, scalar multiply and bias add."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import cu, down, out_half_ulp_rel, up
from oracle import cpu_path as ref
from oracle.quant import bf16_bits, bf16_to_f32, quantize

pytestmark = pytest.mark.gpu


def _special_f32():
    bits = np.array([0x00000000, 0x80000000, 0x3F800000, 0x3F808000, 0x3F818000, 0x3F80C000,
                     0x3F807FFF, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F8000, 0x00000001, 0x807FFFFF,
                     0x00400000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00001, 0x7F800001,
                     0x477FF000, 0x477FE000, 0x33800000, 0x33000001, 0x38800000, 0x387FC000],
                    dtype=np.uint32)
    rng = np.random.default_rng(0)
    rand = rng.integers(0, 2 ** 32, 4000, dtype=np.uint64).astype(np.uint32)
    return np.concatenate([bits, rand]).view(np.float32)


def test_cast_f32_to_bf16_bit_exact():
    x = _special_f32()
    g = cu()
    gt = g.gputensor_from_numpy(x, -1, "bfloat16")
    got = g.gputensor_bits_to_numpy(gt)
    want = bf16_bits(x)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all(np.isnan(bf16_to_f32(got[nan])))
    # the bf16 -> f32 widening is exact
    assert np.array_equal(g.gputensor_to_numpy(gt)[~nan].view(np.uint32),
                          bf16_to_f32(want[~nan]).view(np.uint32))


def test_cast_f32_to_f16_bit_exact():
    x = _special_f32()
    g = cu()
    gt = g.gputensor_from_numpy(x, -1, np.float16)
    got = g.gputensor_bits_to_numpy(gt).view(np.uint16)
    with np.errstate(over="ignore", invalid="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all(np.isnan(got[nan].view(np.float16)))


def test_cast_roundtrip_16bit_exact():
    rng = np.random.default_rng(1)
    x = quantize(rng.standard_normal(10007).astype(np.float32) * 50, "bfloat16")
    assert np.array_equal(down(up(x, "bfloat16")), x)
    h = quantize(rng.standard_normal(10007).astype(np.float32) * 50, "float16")
    assert np.array_equal(down(up(h, "float16")), h)
    g = cu()
    assert np.array_equal(down(g.dev_cast(up(h, "float16"), "bfloat16")), quantize(h, "bfloat16"))


def _softmax_bound(p64, out_dtype):
    rel = out_half_ulp_rel(out_dtype) + 8e-6
    sub = {"float32": 1e-30, "float16": 2.0 ** -25, "bfloat16": 1e-30}[out_dtype]
    return rel * p64 + sub + 1e-9


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("cols", [1, 7, 8, 64, 100, 512, 520, 1024, 2048, 4096, 8192, 8200])
def test_softmax(dtype, cols):
    rng = np.random.default_rng(cols)
    rows = 37
    x = quantize((rng.standard_normal((rows, cols)) * 3).astype(np.float32), dtype)
    scale = 0.125
    p = down(cu().dev_softmax(up(x, dtype), -1, scale))
    p64 = ref.softmax_f64(x, scale)
    err = np.abs(p - p64)
    assert np.all(err <= _softmax_bound(p64, dtype)), float(np.max(err - _softmax_bound(p64, dtype)))
    assert np.allclose(p.astype(np.float64).sum(axis=-1), 1.0, atol=cols * out_half_ulp_rel(dtype) + 1e-5)


def test_softmax_invariants():
    g = cu()
    x = np.full((3, 4096), 2.5, np.float32)
    p = down(g.dev_softmax(up(x, "float32")))
    assert np.allclose(p, 1.0 / 4096, rtol=1e-6)
    x = np.array([[0.0, np.log(2.0)] * 4], np.float32)  # cols = 8
    p = down(g.dev_softmax(up(x, "float32")))
    assert np.allclose(p[0, :2] * 4, [1 / 3, 2 / 3], rtol=1e-6)
    rng = np.random.default_rng(3)
    y = rng.standard_normal((5, 300)).astype(np.float32)
    p1 = down(g.dev_softmax(up(y, "float32")))
    p2 = down(g.dev_softmax(up(y + np.float32(8.0), "float32")))
    assert np.allclose(p1, p2, rtol=2e-5, atol=1e-9)
    with pytest.raises(NotImplementedError):
        g.dev_softmax(up(y, "float32"), 0)


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("op", ["silu", "gelu", "muls"])
@pytest.mark.parametrize("n", [1, 7, 8, 1000, 65536 + 3])
def test_elementwise(dtype, op, n):
    rng = np.random.default_rng(n)
    x = quantize((rng.standard_normal(n) * 4).astype(np.float32), dtype)
    if n > 8:
        x[:6] = quantize(np.array([0.0, -0.0, 30.0, -30.0, 90.0, -90.0], np.float32), dtype)
    g = cu()
    gx = up(x, dtype)
    if op == "silu":
        y, y64 = down(g.dev_silu(gx)), ref.act_f64(x.astype(np.float64), "silu")
    elif op == "gelu":
        y, y64 = down(g.dev_gelu(gx)), ref.act_f64(x.astype(np.float64), "gelu")
    else:
        y, y64 = down(g.dev_muls(gx, -0.3)), x.astype(np.float64) * np.float64(np.float32(-0.3))
    bound = (out_half_ulp_rel(dtype) + 4e-6) * np.abs(y64) + 1e-7 + (2.0 ** -25 if dtype == "float16" else 0)
    err = np.abs(y - y64)
    assert np.all(err <= bound), (op, dtype, float(np.max(err - bound)))


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_bias_add(dtype):
    rng = np.random.default_rng(9)
    c = quantize(rng.standard_normal((33, 70)).astype(np.float32), dtype)
    b = quantize(rng.standard_normal(70).astype(np.float32), dtype)
    g = cu()
    gc = up(c, dtype)
    g.dev_bias_add(gc, up(b, dtype))
    y64 = c.astype(np.float64) + b
    bound = out_half_ulp_rel(dtype) * np.abs(y64) + 1e-30
    assert np.all(np.abs(down(gc) - y64) <= bound)


@pytest.mark.parametrize("n,dtype", [(40_000_001, np.float16), (16_777_219, np.float32), (1001, np.float16)],
                         ids=["80MB-f16-ragged", "64MB-f32-ragged", "small"])
def test_zero_fill(n, dtype):
    """sf_zero over a block that held non-zero data: large fills (64 MB and
    up: non-temporal stores, one workgroup per 512 16-byte stores) and a
    small one, with sizes that leave tail bytes past the last 16-byte store.
    The caching allocator hands the freed block back to the zero fill, so
    every byte the fill misses would still read as one."""
    ones = cu().gputensor_from_numpy(np.ones((n,), np.float32), -1, np.dtype(dtype))
    del ones
    z = cu().zeros((n,), dtype, 0)
    cu().device_synchronize()
    got = cu().gputensor_to_numpy(z)
    assert got.shape == (n,)
    assert np.count_nonzero(got) == 0
