"""Dropout on the device (sf_dropout / dev_dropout / F.dropout / nn.Dropout
and SDPA's dropout_p) against the oracle's restatement (oracle/dropout.py):
the masks bit for bit (this library's Philox4x32-10 stream, pinned there by
the Random123 known-answer vectors), the outputs as x * mask rounded once
into the dtype, and the keep rate against the binomial law of the
reference's rule (_cuda_kernels.cu:1431-1457: keep when u >= p, scale
1 / (1 - p))."""
from __future__ import annotations

import math

import numpy as np
import pytest

from helpers import cu, down, rnd, up
from oracle import cpu_path as ref
from oracle import dropout as D
from oracle.configs import tol_16, tol_fp32
from oracle.quant import quantize

pytestmark = pytest.mark.gpu

DTYPES = ["float32", "float16", "bfloat16"]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [1, 7, 8, 13, 1000, 65536 + 3])
@pytest.mark.parametrize("p", [0.1, 0.5])
def test_dev_dropout_matches_oracle(dtype, n, p):
    rng = np.random.default_rng(n + int(p * 10))
    x = rnd(rng, (n,), 1.0, dtype)
    seed, offset = 0x0123_4567_89AB_CDEF, (1 << 33) + 5  # both words of each
    y, m = cu().dev_dropout(up(x, dtype), p, seed, offset)
    y, m = down(y), down(m)
    y_ref, m_ref = D.dropout(x, p, seed, offset)
    assert np.array_equal(m, quantize(m_ref, dtype))
    assert np.array_equal(y, quantize(y_ref, dtype))


@pytest.mark.parametrize("p", [0.05, 0.3, 0.7])
def test_keep_rate_and_scale(p):
    n = 1 << 20
    x = np.ones(n, np.float32)
    y, m = cu().dev_dropout(up(x, "float32"), p, 99)
    m = down(m)
    dropped = int(np.count_nonzero(m == 0))
    sd = math.sqrt(n * p * (1 - p))
    assert abs(dropped - n * p) < 6 * sd, (dropped, n * p)
    scale = np.float32(1) / (np.float32(1) - np.float32(p))
    assert set(np.unique(m).tolist()) == {0.0, float(scale)}
    assert np.array_equal(down(y), m)


def test_streams_and_edge_cases():
    g = cu()
    x = up(np.arange(1, 4097, dtype=np.float32), "float32")
    a = down(g.dev_dropout(x, 0.5, 5, 0)[1])
    assert np.array_equal(a, down(g.dev_dropout(x, 0.5, 5, 0)[1]))  # same stream, same mask
    assert not np.array_equal(a, down(g.dev_dropout(x, 0.5, 5, 1)[1]))  # next offset
    assert not np.array_equal(a, down(g.dev_dropout(x, 0.5, 6, 0)[1]))  # other seed
    y1, m1 = g.dev_dropout(x, 0.5, 5, 0, False)  # no mask: the same output
    assert m1 is None and np.array_equal(down(y1), down(x) * a)
    y0, m0 = g.dev_dropout(x, 0.0, 5)
    assert np.array_equal(down(y0), down(x)) and np.all(down(m0) == 1.0)
    with pytest.raises(ValueError):
        g.dev_dropout(x, 1.0)
    with pytest.raises(ValueError):
        g.dev_dropout(x, -0.5)
    # in place through the C ABI (x == y), mask not written
    import ctypes
    import os
    lib = ctypes.CDLL(os.path.join(os.path.dirname(g.__file__), "libsfgemm.so"))
    t = up(np.full(1000, 2.0, np.float32), "float32")
    ptr = ctypes.c_void_p(t.data_ptr)
    rc = lib.sf_dropout(ptr, ptr, None, ctypes.c_int64(1000), 0, ctypes.c_float(0.25), ctypes.c_uint64(3),
                        ctypes.c_uint64(4), None)
    assert rc == 0
    g.device_synchronize()
    want, _ = D.dropout(np.full(1000, 2.0, np.float32), 0.25, 3, 4)
    assert np.array_equal(down(t), want)


def test_functional_and_module_dropout():
    import scaffolding_amd as sf
    from scaffolding_amd import nn
    from scaffolding_amd.nn import functional as F
    rng = np.random.default_rng(3)
    x = rnd(rng, (64, 96), 1.0, "bfloat16")
    t = sf.Tensor(x, dtype="bfloat16", device="cuda")
    assert F.dropout(t, 0.3, training=False) is t
    assert F.dropout(t, 0.0) is t
    sf.cuda.manual_seed(1234)
    a = F.dropout(t, 0.3).numpy()
    b = F.dropout(t, 0.3).numpy()
    assert not np.array_equal(a, b)  # successive calls draw successive streams
    sf.cuda.manual_seed(1234)
    assert np.array_equal(F.dropout(t, 0.3).numpy(), a)  # reproducible from the seed
    want, _ = D.dropout(x, 0.3, 1234, 0)
    assert np.array_equal(np.asarray(a, np.float32), quantize(want, "bfloat16"))
    layer = nn.Dropout(0.3)
    sf.cuda.manual_seed(1234)
    assert np.array_equal(layer(t).numpy(), a)
    layer.eval()
    assert layer(t) is t


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_sdpa_dropout_against_oracle(dtype):
    """softmax(scale q k^T) -> dropout (the stream after manual_seed, first
    draw) -> @ v, the reference GPU branch's order (nn/functional.py:314-321),
    against fp64 with the same keep mask."""
    import scaffolding_amd as sf
    from scaffolding_amd.nn import functional as F
    rng = np.random.default_rng(17)
    b, s, d, p = 3, 80, 64, 0.2
    q, k, v = (rnd(rng, (b, s, d), 1.0, dtype) for _ in range(3))
    tq, tk, tv = (sf.Tensor(a, dtype=dtype, device="cuda") for a in (q, k, v))
    sf.cuda.manual_seed(77)
    o = np.asarray(F.scaled_dot_product_attention(tq, tk, tv, dropout_p=p).numpy(), np.float64)
    keep = D.keep(b * s * s, p, 77, 0).reshape(b, s, s)
    scale = 1.0 / math.sqrt(d)
    sc = scale * np.matmul(q.astype(np.float64), np.swapaxes(k, -1, -2).astype(np.float64))
    pr = np.exp(sc - sc.max(-1, keepdims=True))
    pr /= pr.sum(-1, keepdims=True)
    o64 = np.matmul(pr * keep / (1 - p), v.astype(np.float64))
    err = float(np.max(np.abs(o - o64)))
    if dtype == "float32":
        assert err <= 50 * tol_fp32(s) * (1 + float(np.max(np.abs(o64)))), err
    else:
        # scores, probabilities and the dropped probabilities each round
        # into the dtype before PV: a few ulps of the output's scale
        eps = 2.0 ** -8 if dtype == "bfloat16" else 2.0 ** -11
        assert err <= tol_16(s) + 4 * eps * float(np.max(np.abs(v))) / (1 - p), err
    # without dropout the same call takes the fused or unfused path unchanged
    o0 = np.asarray(F.scaled_dot_product_attention(tq, tk, tv).numpy(), np.float64)
    assert float(np.max(np.abs(o0 - ref.sdpa_f64(q, k, v, scale)))) <= tol_16(s) + 2.0 ** -7
