"""BASELINE.json's five configs at full size, on the GPU, to the tolerances
BASELINE.json states:

  fp32       normwise max|y - y_cpu| / max|y_cpu| <= 1e-5 sqrt(K), y_cpu the
             reference's CPU fp32 path (NumPy, oracle.cpu_path)
  bf16/fp16  max|y - y_fp64| <= 2e-2 sqrt(K / 1024), y_fp64 the closed form in
             float64 on the same quantized inputs

Full outputs are checked where the CPU side is cheap; otherwise on sampled
rows (tile edges plus a seeded sample) together with size-independent
properties over every element (row / column checksums for the linear maps,
row sums of the softmax)."""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from helpers import cu, down, sample_rows, up
from oracle import configs as cfg
from oracle import cpu_path as ref

pytestmark = pytest.mark.gpu

# Each check's measured error against its gate; written as JSON to the path
# in SF_PARITY_REPORT (if set) when the module's tests end.
_REPORT = []


@pytest.fixture(scope="module", autouse=True)
def _parity_report():
    yield
    path = os.environ.get("SF_PARITY_REPORT")
    if path and _REPORT:
        with open(path, "w") as f:
            json.dump(_REPORT, f, indent=1)


def _gate(check: str, err: float, tol: float) -> float:
    _REPORT.append({"check": check, "max_err": float(err), "tol": float(tol)})
    return err


def _plan_linear(gx, gw, gb, m, n, k):
    return cu().gemm_plan(1, m, n, k, 1, gx.data_ptr, k, 0, gw.data_ptr, k, 0, n, 0, gx.dtype,
                          epi=1 if gb is not None else 0, ptr_bias=gb.data_ptr if gb is not None else 0)


def test_c1_linear_fp32():
    case = cfg.c1_linear()
    g = cu()
    gy = g.dev_linear_forward(up(case.x, "float32"), up(case.w, "float32"), up(case.b, "float32"))
    assert gy.shape == (64, 512) and gy.dtype == np.float32
    y = down(gy)
    y_cpu = ref.linear(case.x, case.w, case.b)
    err = _gate("C1 fp32 linear, normwise vs CPU fp32", cfg.normwise_err(y, y_cpu), cfg.tol_fp32(512))
    assert err <= cfg.tol_fp32(512), err
    # and against the exact value
    assert cfg.normwise_err(y, ref.linear_f64(case.x, case.w, case.b)) <= cfg.tol_fp32(512)


@pytest.mark.parametrize("n", [1024, 2048, 4096])
def test_c2_matmul_fp32(n):
    a, b = cfg.c2_matmul(n)
    g = cu()
    y = down(g.dev_matmul(up(a, "float32"), up(b, "float32")))
    assert y.shape == (n, n)
    rows = sample_rows(n, 192, seed=n, tile=128)
    y_cpu = ref.matmul(a[rows], b)  # the reference CPU path on these rows
    err = _gate("C2 fp32 matmul %d, normwise vs CPU fp32 (sampled rows)" % n, cfg.normwise_err(y[rows], y_cpu),
                cfg.tol_fp32(n))
    assert err <= cfg.tol_fp32(n), err
    # every row and column: checksums against fp64
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    rs = y.astype(np.float64).sum(axis=1)
    cs = y.astype(np.float64).sum(axis=0)
    bound_r = cfg.tol_fp32(n) * np.abs(a64) @ np.abs(b64).sum(axis=1)
    bound_c = cfg.tol_fp32(n) * np.abs(a64).sum(axis=0) @ np.abs(b64)
    assert np.all(np.abs(rs - a64 @ b64.sum(axis=1)) <= bound_r)
    assert np.all(np.abs(cs - a64.sum(axis=0) @ b64) <= bound_c)


@pytest.mark.parametrize("m", [1, 16, 4096])
def test_c3_linear_silu_bf16(m):
    case = cfg.c3_linear(m)
    k, n = case.x.shape[1], case.w.shape[0]
    g = cu()
    gx, gw, gb = up(case.x, "bfloat16"), up(case.w, "bfloat16"), up(case.b, "bfloat16")
    plan = _plan_linear(gx, gw, gb, m, n, k)
    assert plan.startswith("gemm skinny" if m <= 16 else "gemm nt 256x256"), plan
    gy = g.dev_linear_forward(gx, gw, gb, "silu")
    assert gy.shape == (m, n) and gy.dtype == g.BFLOAT16
    y = down(gy)
    rows = np.arange(m) if m <= 16 else sample_rows(m, 256, seed=2)
    y64 = ref.linear_f64(case.x[rows], case.w, case.b, "silu")
    err = _gate("C3 bf16 linear+bias+SiLU M=%d, abs vs fp64" % m, cfg.abs_err(y[rows], y64), cfg.tol_16(k))
    assert err <= cfg.tol_16(k), err
    assert np.all(np.isfinite(y))


def test_c4_attention_fp16():
    q, k, v, scale = cfg.c4_attention()
    g = cu()
    gq, gk, gv = up(q, "float16"), up(k, "float16"), up(v, "float16")
    bh, s, d = q.shape
    # QK^T with the 1/8 scale folded into the epilogue, fp16 scores.
    gs = g.dev_batched_matmul_nt(gq, gk, scale)
    assert gs.shape == (bh, s, s) and gs.dtype == np.float16
    scores = g.gputensor_to_numpy(gs)  # fp16 host copy, 2 GB
    rng = np.random.default_rng(33)
    heads = np.unique(np.r_[0, bh - 1, rng.choice(bh, 4, replace=False)])
    rows = sample_rows(s, 24, seed=34)
    for h in heads:
        s64 = scale * (q[h, rows].astype(np.float64) @ k[h].astype(np.float64).T)
        err = _gate("C4 fp16 alpha-scaled QK^T head %d, abs vs fp64" % h,
                    cfg.abs_err(scores[h, rows].astype(np.float32), s64), cfg.tol_16(d))
        assert err <= cfg.tol_16(d), (h, err)
    # softmax over every row: rows sum to one (fp16 output spacing bound)
    gp = g.dev_softmax(gs, -1)
    del scores, gs
    probs = g.gputensor_to_numpy(gp)
    sums = probs.astype(np.float64).sum(axis=-1)
    assert np.all(np.abs(sums - 1.0) <= s * 2.0 ** -11 * (1.0 / s) * 4 + 2e-3), float(np.max(np.abs(sums - 1)))
    del probs, gp
    # end-to-end SDPA output against fp64 softmax(scale q k^T) v: the
    # three-launch path and the fused kernel
    for fn in (g.dev_sdpa_unfused, g.dev_scaled_dot_product_attention):
        go = fn(gq, gk, gv, scale)
        assert go.shape == (bh, s, d) and go.dtype == np.float16
        o = g.gputensor_to_numpy(go).astype(np.float32)
        del go
        for h in heads:
            o64 = ref.sdpa_f64(q[h:h + 1, rows], k[h:h + 1], v[h:h + 1], scale)[0]
            err = _gate("C4 fp16 SDPA (%s) head %d, abs vs fp64" % (fn.__name__, h), cfg.abs_err(o[h, rows], o64),
                        cfg.tol_16(s))
            assert err <= cfg.tol_16(s), (fn.__name__, h, err)


@pytest.mark.parametrize("proj", list(cfg.C5_PROJ))
def test_c5_dit_projections_bf16(proj):
    case = cfg.c5_projection(proj)
    k, n = case.x.shape[1], case.w.shape[0]
    m = case.x.shape[0]
    g = cu()
    gx, gw = up(case.x, "bfloat16"), up(case.w, "bfloat16")
    gb = up(case.b, "bfloat16") if case.b is not None else None
    gy = g.dev_linear_forward(gx, gw, gb, case.act)
    assert gy.shape == (m, n)
    y = down(gy)
    rows = sample_rows(m, 192, seed=4 + k + n)
    # the ragged last 256-row tile (17664..17775) is checked against fp64 too
    last = (m - 1) // 256 * 256
    assert np.count_nonzero(rows >= last) >= 4 and rows[-1] == m - 1
    y64 = ref.linear_f64(case.x[rows], case.w, case.b, case.act)
    err = _gate("C5 bf16 %s, abs vs fp64 (sampled rows)" % proj, cfg.abs_err(y[rows], y64), cfg.tol_16(k))
    assert err <= cfg.tol_16(k), err
    if case.act is None:
        # every row: y . 1 = x . (W^T 1) + sum(b), fp64 on the quantized inputs
        w1 = case.w.astype(np.float64).sum(axis=0)
        rs64 = case.x.astype(np.float64) @ w1 + (case.b.astype(np.float64).sum() if case.b is not None else 0.0)
        rs = y.astype(np.float64).sum(axis=1)
        assert np.all(np.abs(rs - rs64) <= n * cfg.tol_16(k)), float(np.max(np.abs(rs - rs64)))
