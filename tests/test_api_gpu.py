"""The Python API surface of the path on the GPU, against the oracle:
``Tensor`` / ``matmul`` / ``@`` (reference tensor.py:1480-1526), ``matmul_nt``
(tensor.py:1529-1539), ``nn.Linear`` (nn/layers.py:83-146), ``F.linear``
(nn/functional.py:374-395), ``F.silu`` / ``F.gelu`` / ``F.softmax``
(nn/functional.py:37-145) and ``F.scaled_dot_product_attention``
(nn/functional.py:298-369), at BASELINE.json's config shapes.

Tolerances are BASELINE.json's: fp32 normwise <= 1e-5 sqrt(K) against the
reference's CPU fp32 path, 16-bit max abs <= 2e-2 sqrt(K / 1024) against
fp64 on the quantized inputs.  Every result is also checked for the
reference's output shape (x.shape[:-1] + (N,), a.shape[:-2] + (M, N)),
dtype and a C-contiguous host view, and the API's refusals are checked.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import scaffolding_amd as sf
from scaffolding_amd.nn import functional as F
from helpers import check_bound, gemm_bound, rnd, sample_rows
from oracle import configs as cfg
from oracle import cpu_path as ref

pytestmark = pytest.mark.gpu


def dev(x, dtype="float32"):
    return sf.Tensor(x, dtype=dtype, device="cuda")


def host(t: sf.Tensor) -> np.ndarray:
    a = t.numpy()
    assert a.flags.c_contiguous
    return np.asarray(a, np.float32)


def test_c1_nn_linear_module_fp32():
    """C1 through the module: nn.Linear(512, 512) with the config's W and b
    loaded by load_state_dict, called on a cuda Tensor."""
    case = cfg.c1_linear()
    lin = sf.nn.Linear(512, 512, device="cuda", dtype="float32")
    lin.load_state_dict({"weight": case.w, "bias": case.b})
    y = lin(dev(case.x))
    assert y.shape == (64, 512) and y.dtype is sf.float32 and y.is_cuda
    yh = host(y)
    y_cpu = ref.linear(case.x, case.w, case.b)
    assert cfg.normwise_err(yh, y_cpu) <= cfg.tol_fp32(512)
    # Leading dims flatten as the reference's dev_linear_forward does
    y3 = lin(dev(case.x.reshape(4, 16, 512)))
    assert y3.shape == (4, 16, 512)
    assert np.array_equal(host(y3).reshape(64, 512), yh)


@pytest.mark.parametrize("op", ["matmul", "method", "operator"])
def test_c2_matmul_2d_fp32(op):
    """C2 at n = 1024 through sf.matmul, Tensor.matmul and @: the 2-D branch
    (dev_matmul)."""
    n = 1024
    a, b = cfg.c2_matmul(n)
    ta, tb = dev(a), dev(b)
    y = {"matmul": lambda: sf.matmul(ta, tb), "method": lambda: ta.matmul(tb),
         "operator": lambda: ta @ tb}[op]()
    assert y.shape == (n, n) and y.dtype is sf.float32
    yh = host(y)
    rows = sample_rows(n, 128, seed=n, tile=128)
    assert cfg.normwise_err(yh[rows], ref.matmul(a[rows], b)) <= cfg.tol_fp32(n)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("case", ["a3d_b2d", "a2d_b3d", "both3d", "a4d_b2d"])
def test_matmul_batched_broadcast(dtype, case):
    """The >= 3-D branch (dev_batched_matmul) with np.matmul's broadcast of
    a 2-D operand, against fp64 np.matmul on the same values."""
    rng = np.random.default_rng(len(case) + len(dtype))
    m, k, n = 70, 96, 50
    shapes = {"a3d_b2d": ((3, m, k), (k, n)), "a2d_b3d": ((m, k), (3, k, n)),
              "both3d": ((3, m, k), (3, k, n)), "a4d_b2d": ((2, 3, m, k), (k, n))}[case]
    a = rnd(rng, shapes[0], 1.0, dtype)
    b = rnd(rng, shapes[1], 1.0, dtype)
    y = dev(a, dtype) @ dev(b, dtype)
    want_shape = np.matmul(a, b).shape
    assert y.shape == want_shape
    assert y.dtype is getattr(sf, dtype)
    y64 = np.matmul(a.astype(np.float64), b.astype(np.float64))
    if dtype == "float32":
        assert cfg.normwise_err(host(y), y64) <= cfg.tol_fp32(k)
    else:
        # N(0, 1) operands give |y| up to ~30, far above BASELINE's unit-scale
        # outputs: the elementwise bound (fp32 accumulation plus one
        # rounding into the dtype) is the meaningful one here.
        absprod = np.matmul(np.abs(a).astype(np.float64), np.abs(b).astype(np.float64))
        check_bound(host(y), y64, gemm_bound(y64, absprod, k, dtype), "batched %s %s" % (case, dtype))


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("case", ["vec_mat", "mat_vec", "vec_vec", "batch_vec", "vec_batch"])
def test_matmul_1d_operands(case, dtype):
    """1-D operands follow np.matmul (the reference's host branch,
    tensor.py:1494-1497): a vector on the left is a row, on the right a
    column, and that axis is dropped; the product runs on the device."""
    rng = np.random.default_rng(["vec_mat", "mat_vec", "vec_vec", "batch_vec", "vec_batch"].index(case) * 2
                                + (dtype == "bfloat16") + 61)
    m, k, n = 37, 520, 70
    shapes = {"vec_mat": ((k,), (k, n)), "mat_vec": ((m, k), (k,)), "vec_vec": ((k,), (k,)),
              "batch_vec": ((3, m, k), (k,)), "vec_batch": ((k,), (2, k, n))}[case]
    a = rnd(rng, shapes[0], 1.0, dtype)
    b = rnd(rng, shapes[1], 1.0, dtype)
    y = dev(a, dtype) @ dev(b, dtype)
    y64 = np.matmul(a.astype(np.float64), b.astype(np.float64))
    assert y.shape == y64.shape, (y.shape, y64.shape)
    assert y.dtype is getattr(sf, dtype)
    absprod = np.matmul(np.abs(a).astype(np.float64), np.abs(b).astype(np.float64))
    got = np.asarray(host(y), dtype=np.float64)
    check_bound(got.reshape(-1), y64.reshape(-1), gemm_bound(y64, absprod, k, dtype).reshape(-1),
                "1-D %s %s" % (case, dtype))


def test_matmul_refusals():
    a = dev(np.ones((4, 8), np.float32))
    with pytest.raises(ValueError):
        sf.matmul(a, dev(np.ones((7,), np.float32)))  # the vector's length is not K
    with pytest.raises(RuntimeError, match="GPU only"):
        sf.matmul(sf.Tensor(np.ones((4, 8), np.float32)), sf.Tensor(np.ones((8, 2), np.float32)))
    with pytest.raises(ValueError):
        a @ dev(np.ones((7, 2), np.float32))  # inner dims differ


def test_c4_matmul_nt_alpha_fp16():
    """C4's Q K^T through sf.matmul_nt (3-D: dev_batched_matmul_nt) with the
    1/8 scale as alpha; sampled heads and rows against fp64."""
    q, k, _, scale = cfg.c4_attention()
    bh, s, d = q.shape
    tq, tk = dev(q, "float16"), dev(k, "float16")
    t = sf.matmul_nt(tq, tk, scale)
    assert t.shape == (bh, s, s) and t.dtype is sf.float16
    scores = t.numpy()
    assert scores.flags.c_contiguous and scores.dtype == np.float16
    del t
    rng = np.random.default_rng(41)
    heads = np.unique(np.r_[0, bh - 1, rng.choice(bh, 3, replace=False)])
    rows = sample_rows(s, 16, seed=42)
    for h in heads:
        s64 = scale * (q[h, rows].astype(np.float64) @ k[h].astype(np.float64).T)
        assert cfg.abs_err(scores[h, rows].astype(np.float32), s64) <= cfg.tol_16(d), h
    # the 2-D branch (dev_matmul_nt), default alpha
    t2 = sf.matmul_nt(dev(q[0], "float16"), dev(k[0], "float16"))
    assert t2.shape == (s, s)
    s64 = q[0, rows].astype(np.float64) @ k[0].astype(np.float64).T
    absprod = np.abs(q[0, rows]).astype(np.float64) @ np.abs(k[0]).astype(np.float64).T
    check_bound(host(t2)[rows], s64, gemm_bound(s64, absprod, d, "float16"), "matmul_nt 2-D")


@pytest.mark.parametrize("fused", [False, True])
def test_c3_f_linear_then_silu_bf16(fused):
    """C3 at M = 16 through F.linear: as the reference's caller does it
    (F.linear, then F.silu on the result) and with the fused activation."""
    case = cfg.c3_linear(16)
    tx, tw, tb = dev(case.x, "bfloat16"), dev(case.w, "bfloat16"), dev(case.b, "bfloat16")
    if fused:
        y = F.linear(tx, tw, tb, activation="silu")
    else:
        z = F.linear(tx, tw, tb)
        assert z.shape == (16, 11008) and z.dtype is sf.bfloat16
        y = F.silu(z)
    assert y.shape == (16, 11008) and y.dtype is sf.bfloat16
    y64 = ref.linear_f64(case.x, case.w, case.b, "silu")
    assert cfg.abs_err(host(y), y64) <= cfg.tol_16(4096)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_f_gelu_silu_softmax(dtype):
    """Elementwise ops and the row softmax against the fp64 closed forms
    (one rounding into the dtype, plus fp32 arithmetic)."""
    rng = np.random.default_rng(5)
    x = rnd(rng, (33, 257), 3.0, dtype)
    eps = {"float32": 2.0 ** -23, "bfloat16": 2.0 ** -8}[dtype]
    t = dev(x, dtype)
    for fn, f64 in ((F.gelu, lambda v: ref.act_f64(v, "gelu_tanh")), (F.silu, lambda v: ref.act_f64(v, "silu"))):
        y = fn(t)
        assert y.shape == x.shape and y.dtype is getattr(sf, dtype)
        want = f64(x.astype(np.float64))
        assert np.all(np.abs(host(y) - want) <= (eps + 4e-6) * np.abs(want) + 1e-6)
    p = F.softmax(t, dim=-1)
    assert p.shape == x.shape
    want = ref.softmax_f64(x)
    assert np.all(np.abs(host(p) - want) <= (eps + 1e-5) * want + 1e-7)
    with pytest.raises(NotImplementedError):
        F.gelu(t, approximate="none")


def test_c4_f_scaled_dot_product_attention_fp16():
    """C4 through F.scaled_dot_product_attention: default scale 1/sqrt(64),
    sampled heads and rows against fp64 softmax(q k^T / 8) v."""
    q, k, v, scale = cfg.c4_attention()
    bh, s, d = q.shape
    o = F.scaled_dot_product_attention(dev(q, "float16"), dev(k, "float16"), dev(v, "float16"))
    assert o.shape == (bh, s, d) and o.dtype is sf.float16
    oh = host(o)
    assert np.all(np.isfinite(oh))
    rng = np.random.default_rng(43)
    heads = np.unique(np.r_[0, bh - 1, rng.choice(bh, 3, replace=False)])
    rows = sample_rows(s, 24, seed=44)
    for h in heads:
        o64 = ref.sdpa_f64(q[h:h + 1, rows], k[h:h + 1], v[h:h + 1], 1.0 / math.sqrt(d))[0]
        assert cfg.abs_err(oh[h, rows], o64) <= cfg.tol_16(s), h
    assert scale == 1.0 / math.sqrt(d)


def test_sdpa_refusals_and_explicit_scale():
    rng = np.random.default_rng(6)
    q = rnd(rng, (2, 40, 64), 1.0, "bfloat16")
    tq = dev(q, "bfloat16")
    with pytest.raises(ValueError, match="broadcast"):  # a (2, 40, 64) mask on (2, 40, 40) scores
        F.scaled_dot_product_attention(tq, tq, tq, attn_mask=tq)
    with pytest.raises(ValueError, match="dropout_p"):
        F.scaled_dot_product_attention(tq, tq, tq, dropout_p=1.0)
    with pytest.raises(RuntimeError, match="GPU only"):
        F.scaled_dot_product_attention(sf.Tensor(q), sf.Tensor(q), sf.Tensor(q))
    o = F.scaled_dot_product_attention(tq, tq, tq, scale=0.3)
    o64 = ref.sdpa_f64(q, q, q, 0.3)
    assert cfg.abs_err(host(o), o64) <= cfg.tol_16(40) + 2 * 2.0 ** -8 * float(np.max(np.abs(q)))


def test_north_star_linear_bias_bf16_4096():
    """The headline workload itself, x[4096, 4096] W[4096, 4096]^T + b in
    bf16 through nn.Linear: sampled rows against fp64 and every row's sum
    (y 1 = x (W^T 1) + sum b) against fp64."""
    m = n = k = 4096
    rng = np.random.default_rng(12)
    x = rnd(rng, (m, k), 1.0, "bfloat16")
    w = rnd(rng, (n, k), 0.02, "bfloat16")
    b = rnd(rng, (n,), 0.01, "bfloat16")
    lin = sf.nn.Linear(k, n, device="cuda", dtype="bfloat16")
    lin.load_state_dict({"weight": w, "bias": b})
    y = lin(dev(x, "bfloat16"))
    assert y.shape == (m, n) and y.dtype is sf.bfloat16
    yh = host(y)
    rows = sample_rows(m, 192, seed=13)
    y64 = ref.linear_f64(x[rows], w, b)
    assert cfg.abs_err(yh[rows], y64) <= cfg.tol_16(k)
    rs64 = x.astype(np.float64) @ w.astype(np.float64).sum(axis=0) + b.astype(np.float64).sum()
    rs = yh.astype(np.float64).sum(axis=1)
    assert np.all(np.abs(rs - rs64) <= n * cfg.tol_16(k)), float(np.max(np.abs(rs - rs64)))


def test_runtime_module_surface():
    """``sf.cuda`` (reference cuda/__init__.py:45-303) and
    ``sf.backends.cuda.matmul.allow_tf32`` (reference backends/cuda.py:20-35)
    on the device: availability and properties, events timing a GEMM,
    the caching allocator's live and pooled bytes as a tensor comes and
    goes, and the tf32 flag (recorded, the fp32 GEMM bit-identical either
    way)."""
    assert sf.cuda.is_available() and sf.cuda.device_count() >= 1
    sf.cuda.set_device(0)
    assert sf.cuda.current_device() == 0
    props = sf.cuda.get_device_properties(0)
    assert props["arch"].startswith("gfx950") and props["multi_processor_count"] > 0
    assert props["total_memory"] > (1 << 34)
    assert isinstance(sf.cuda.get_device_name(0), str)

    rng = np.random.default_rng(5)
    a = dev(rng.standard_normal((1024, 1024), dtype=np.float32))
    b = dev(rng.standard_normal((1024, 1024), dtype=np.float32))
    e0, e1 = sf.cuda.Event(), sf.cuda.Event()
    e0.record()
    c = sf.matmul(a, b)
    e1.record()
    e1.synchronize()
    assert 0.0 < e0.elapsed_time(e1) < 1000.0

    sf.cuda.synchronize()
    live0 = sf.cuda.memory_allocated()
    t = dev(np.zeros((1024, 1024), np.float32))  # 4 MiB
    assert sf.cuda.memory_allocated() >= live0 + (4 << 20)
    pooled0 = sf.cuda.memory_stats()["pooled_bytes"]
    del t
    assert sf.cuda.memory_allocated() <= live0 + (1 << 20)
    assert sf.cuda.memory_stats()["pooled_bytes"] >= pooled0 + (4 << 20)  # the freed block is pooled
    sf.cuda.empty_cache()
    assert sf.cuda.memory_stats()["pooled_bytes"] == 0

    ref_bits = host(c).view(np.uint32).copy()
    sf.backends.cuda.matmul.allow_tf32 = True
    try:
        assert sf.backends.cuda.matmul.allow_tf32 is True
        c2 = sf.matmul(a, b)
    finally:
        sf.backends.cuda.matmul.allow_tf32 = False
    assert sf.backends.cuda.matmul.allow_tf32 is False
    assert np.array_equal(host(c2).view(np.uint32), ref_bits)
