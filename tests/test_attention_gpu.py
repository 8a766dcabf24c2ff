"""Fused attention (sf_attention) on the GPU against the fp64 closed form
softmax(scale * q k^T) v on the quantized inputs (oracle.cpu_path.sdpa_f64),
with the three-launch path as a second witness; ragged query counts, batch
dims, both 16-bit dtypes, the fallback shapes and the ABI's refusals."""
from __future__ import annotations

import ctypes
import math
import os

import numpy as np
import pytest

from helpers import cu, quantize, rnd, up
from oracle.configs import tol_16

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def sdpa64(q, k, v, scale):
    """fp64 softmax(scale q k^T) v over the last two dims."""
    q64, k64, v64 = (a.astype(np.float64) for a in (q, k, v))
    s = scale * (q64 @ np.swapaxes(k64, -1, -2))
    s -= s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return p @ v64


def down(gt):
    return cu().gputensor_to_numpy(gt).astype(np.float32)


EPS = {"float16": 2.0 ** -11, "bfloat16": 2.0 ** -8}


def bound(q, k, v, scale, dtype, unfused=False):
    """BASELINE's 16-bit tolerance at K = Sk plus the rounding this op adds
    beyond one GEMM: P rounded to the input dtype (relative eps each, moving
    o by <= eps * max|v|), the output rounding (<= eps * max|o| <= eps *
    max|v|), and on the three-launch path the scores rounded before the
    softmax (|d p| <= p * 2 eps |s|, so <= 2 eps max|s| max|v|)."""
    eps = EPS[dtype]
    vmax = float(np.max(np.abs(v)))
    b = tol_16(k.shape[-2]) + 2 * eps * vmax
    if unfused:
        smax = float(np.max(np.abs(scale * (q.astype(np.float64) @ np.swapaxes(k.astype(np.float64), -1, -2)))))
        b += 2 * eps * smax * vmax
    return b


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("shape", [(1, 256, 64), (3, 300, 128), (2, 17, 320), (4, 513, 64)],
                         ids=lambda s: "x".join(map(str, s)))
def test_fused_attention_matches_fp64(dtype, shape):
    b, sq, sk = shape
    rng = np.random.default_rng(sq + 7 * sk + b)
    q = rnd(rng, (b, sq, 64), 1.0, dtype)
    k = rnd(rng, (b, sk, 64), 1.0, dtype)
    v = rnd(rng, (b, sk, 64), 1.0, dtype)
    scale = 0.125
    g = cu()
    gq, gk, gv = up(q, dtype), up(k, dtype), up(v, dtype)
    o = down(g.dev_scaled_dot_product_attention(gq, gk, gv, scale))
    o64 = sdpa64(q, k, v, scale)
    err = float(np.max(np.abs(o - o64)))
    assert err <= bound(q, k, v, scale, dtype), err
    # the three-launch path agrees to its own bound
    o3 = down(g.dev_sdpa_unfused(gq, gk, gv, scale))
    err3 = float(np.max(np.abs(o3 - o64)))
    assert err3 <= bound(q, k, v, scale, dtype, unfused=True), err3


def test_fused_attention_large_scores_and_leading_dims():
    """Scores of magnitude ~50 (exp2 range, running-max correction across
    key blocks: the maximum sits in a late block) and (2, 3, S, 64) inputs."""
    rng = np.random.default_rng(9)
    q = rnd(rng, (2, 3, 130, 64), 1.0, "float16")
    k = rnd(rng, (2, 3, 192, 64), 1.0, "float16")
    k[:, :, 150] = q[:, :, 0:1].mean(axis=2) * 6  # one late key dominates some rows
    k = k.astype(np.float16).astype(np.float32)
    v = rnd(rng, (2, 3, 192, 64), 1.0, "float16")
    g = cu()
    o = down(g.dev_scaled_dot_product_attention(up(q, "float16"), up(k, "float16"), up(v, "float16"), 1.0))
    o64 = sdpa64(q, k, v, 1.0)
    assert o.shape == (2, 3, 130, 64)
    assert np.all(np.isfinite(o))
    assert float(np.max(np.abs(o - o64))) <= bound(q, k, v, 1.0, "float16")


@pytest.mark.parametrize("dtype,scale,qmul,kmul", [
    ("float16", 0.6, 1.0, 1.0),     # scale log2 e = 0.87: Q pre-scaled in registers
    ("float16", 0.125, 3.0, 3.0),   # pre-scaled, scores of magnitude ~50 from larger inputs
    ("bfloat16", 0.125, 1.0, 1.0),  # pre-scaled
    ("bfloat16", 0.125, 3.0, 3.0),  # pre-scaled, large scores: Q's bf16 rounding shows
    ("bfloat16", 1.0, 1.0, 1.0),    # scale log2 e = 1.44: the FMA path
    ("float16", 2.0, 1e4, 1e-4),    # scale log2 e = 2.9: |Q| up to ~4e4 would overflow fp16 if pre-scaled
], ids=["f16-prescaled", "f16-prescaled-large", "bf16-prescaled", "bf16-prescaled-large", "bf16-fma-path",
        "f16-fma-path"])
def test_prescaled_and_fma_exponent_paths(dtype, scale, qmul, kmul):
    """The two ways the kernel forms x = s scale log2 e - m (Q pre-scaled
    with -m as the score MFMAs' C operand, or one FMA per score), with large
    scores that need the running-maximum raise (a late key dominates).  The
    pre-scaled path rounds q scale log2 e into the dtype: each exponent then
    moves by up to eps sum_d |q_d k_d| scale log2 e, which the bound adds
    (the FMA path computes the exponents from exact products in fp32)."""
    rng = np.random.default_rng(int(scale * 10) + (dtype == "bfloat16"))
    q = quantize((rng.standard_normal((2, 200, 64)) * qmul).astype(np.float32), dtype)
    k = rng.standard_normal((2, 320, 64)).astype(np.float32)
    k[:, 290] = q[:, 0:1].mean(axis=1) / qmul * 4  # one late key dominates some rows
    k = quantize(k * kmul, dtype)
    v = rnd(rng, (2, 320, 64), 1.0, dtype)
    g = cu()
    o = down(g.dev_scaled_dot_product_attention(up(q, dtype), up(k, dtype), up(v, dtype), scale))
    o64 = sdpa64(q, k, v, scale)
    assert np.all(np.isfinite(o))
    b = bound(q, k, v, scale, dtype)
    if scale * math.log2(math.e) <= 1.0:
        # |d x| <= eps_Q * scale log2 e * max_k sum_d |q_d k_d| moves each
        # weight by a factor 2^dx and the output by <= (2^dx - 1) 2 max|v|
        absdot = np.abs(q.astype(np.float64)) @ np.swapaxes(np.abs(k.astype(np.float64)), -1, -2)
        dx = EPS[dtype] * scale * math.log2(math.e) * float(np.max(absdot))
        b += (2.0 ** dx - 1.0) * 2 * float(np.max(np.abs(v)))
    assert float(np.max(np.abs(o - o64))) <= b


@pytest.mark.parametrize("shape", [(2, 40, 100, 64), (1, 64, 64, 32), (1, 33, 128, 80)],
                         ids=lambda s: "x".join(map(str, s)))
def test_other_shapes(shape):
    """Sk = 100 (fused, masked tail), head size 32 (fused on 64-wide tiles)
    and 80 (three-launch path)."""
    b, sq, sk, d = shape
    rng = np.random.default_rng(3)
    q = rnd(rng, (b, sq, d), 1.0, "bfloat16")
    k = rnd(rng, (b, sk, d), 1.0, "bfloat16")
    v = rnd(rng, (b, sk, d), 1.0, "bfloat16")
    g = cu()
    o = down(g.dev_scaled_dot_product_attention(up(q, "bfloat16"), up(k, "bfloat16"), up(v, "bfloat16"), None))
    o64 = sdpa64(q, k, v, 1.0 / np.sqrt(d))
    assert float(np.max(np.abs(o - o64))) <= bound(q, k, v, 1.0 / np.sqrt(d), "bfloat16", unfused=True)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("d", [8, 16, 32, 48, 56])
def test_fused_small_head_sizes_ignore_columns_past_d(dtype, d):
    """Head sizes below 64 run fused on 64-wide tiles.  Q, K and V are stored
    with row stride 64 and NaN in every column past D (inside the same
    allocation), and O's columns past D hold a sentinel: the output must be
    finite, match fp64 over the first D columns, and leave the sentinel
    columns untouched (d past D is neither read nor written)."""
    so = ctypes.CDLL(os.path.join(ROOT, "scaffolding_amd", "libsfgemm.so"))
    I64, P = ctypes.c_int64, ctypes.c_void_p
    b, sq, sk = 2, 130, 177
    rng = np.random.default_rng(100 + d)
    q = rnd(rng, (b, sq, d), 1.0, dtype)
    k = rnd(rng, (b, sk, d), 1.0, dtype)
    v = rnd(rng, (b, sk, d), 1.0, dtype)

    def padded(a):
        out = np.full(a.shape[:-1] + (64,), np.nan, np.float32)
        out[..., :d] = a
        return out
    gq, gk, gv = up(padded(q), dtype), up(padded(k), dtype), up(padded(v), dtype)
    go = up(np.full((b, sq, 64), 7.0, np.float32), dtype)
    scale = 1.0 / np.sqrt(d)
    rc = so.sf_attention(P(gq.data_ptr), I64(64), I64(sq * 64), P(gk.data_ptr), I64(64), I64(sk * 64),
                         P(gv.data_ptr), I64(64), I64(sk * 64), P(go.data_ptr), I64(64), I64(sq * 64),
                         I64(b), I64(sq), I64(sk), I64(d), ctypes.c_float(scale), 2 if dtype == "bfloat16" else 1,
                         None)
    assert rc == 0
    cu().device_synchronize()
    o = down(go)
    assert np.all(o[..., d:] == 7.0), "columns past the head size were written"
    assert np.all(np.isfinite(o[..., :d]))
    o64 = sdpa64(q, k, v, scale)
    assert float(np.max(np.abs(o[..., :d] - o64))) <= bound(q, k, v, scale, dtype)
    # and through the tensor entry point (contiguous rows of D)
    o2 = down(cu().dev_scaled_dot_product_attention(up(q, dtype), up(k, dtype), up(v, dtype), None))
    assert float(np.max(np.abs(o2 - o64))) <= bound(q, k, v, scale, dtype)


def test_abi_refusals():
    so = ctypes.CDLL(os.path.join(ROOT, "scaffolding_amd", "libsfgemm.so"))
    so.sf_last_error.restype = ctypes.c_char_p
    I64, P = ctypes.c_int64, ctypes.c_void_p
    # 128 rows: every call below stays inside the buffer (sk <= 128)
    x = up(np.zeros((1, 128, 64), np.float32), "float16")
    p = P(x.data_ptr)

    def call(d=64, sk=64, dt=1, ld=64, scale=1.0):
        return so.sf_attention(p, I64(ld), I64(0), p, I64(ld), I64(0), p, I64(ld), I64(0), p, I64(ld), I64(0),
                               I64(1), I64(64), I64(sk), I64(d), ctypes.c_float(scale), dt, None)
    assert call() == 0
    assert call(sk=96) == 0  # a partial last key block is masked
    assert call(d=32) == 0  # head sizes below 64 run on 64-wide tiles
    assert call(d=72) == -3 and b"head size" in so.sf_last_error()
    assert call(d=36) == -3 and b"head size" in so.sf_last_error()
    assert call(scale=0.0) == -3 and b"scale" in so.sf_last_error()
    assert call(dt=0) == -3 and b"16-bit" in so.sf_last_error()
    assert call(ld=63) == -2
    cu().device_synchronize()


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("parts", [2, 3, 16])
@pytest.mark.parametrize("shape", [(2, 300, 1000, 64), (1, 513, 4095, 64), (3, 130, 1090, 32)],
                         ids=lambda s: "x".join(map(str, s)))
def test_split_key_ranges_match_fp64_and_unsplit(dtype, parts, shape):
    """Every work item split into `parts` key ranges (the attn_parts test hook),
    merged by the combine kernel: matches fp64 to the same bound as the
    unsplit kernel, and the unsplit output to twice the output rounding
    plus P's rounding.  One key far past the first part's range dominates
    some rows, so the parts' row references m differ by large amounts and
    the combine's weights 2^(m_p - M) span a wide range; Sk ragged (last
    part masked), D = 32 (columns past D not stored)."""
    b, sq, sk, d = shape
    rng = np.random.default_rng(sq + sk + parts)
    q = rnd(rng, (b, sq, d), 1.0, dtype)
    k = rnd(rng, (b, sk, d), 1.0, dtype)
    v = rnd(rng, (b, sk, d), 1.0, dtype)
    k[:, sk - 70] = q[:, 0:8].mean(axis=1) * 5
    k = quantize(k, dtype)
    g = cu()
    gq, gk, gv = up(q, dtype), up(k, dtype), up(v, dtype)
    scale = 1.0 / np.sqrt(d)
    o1 = down(g.dev_scaled_dot_product_attention(gq, gk, gv, scale))
    g._set_test_hooks(attn_parts=parts)
    try:
        o = down(g.dev_scaled_dot_product_attention(gq, gk, gv, scale))
    finally:
        g._set_test_hooks()
    o64 = sdpa64(q, k, v, scale)
    assert np.all(np.isfinite(o))
    assert float(np.max(np.abs(o - o64))) <= bound(q, k, v, scale, dtype)
    vmax = float(np.max(np.abs(v)))
    assert float(np.max(np.abs(o - o1))) <= 4 * EPS[dtype] * vmax


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_split_plan_on_a_short_launch(dtype):
    """One head, 1024 query rows, 2048 keys: 4 work items on 2 x CUs slots,
    so the plan splits each into 4 key ranges of 8 blocks (no test hook)."""
    rng = np.random.default_rng(21)
    q = rnd(rng, (1, 1024, 64), 1.0, dtype)
    k = rnd(rng, (1, 2048, 64), 1.0, dtype)
    v = rnd(rng, (1, 2048, 64), 1.0, dtype)
    g = cu()
    o = down(g.dev_scaled_dot_product_attention(up(q, dtype), up(k, dtype), up(v, dtype), 0.125))
    assert float(np.max(np.abs(o - sdpa64(q, k, v, 0.125)))) <= bound(q, k, v, 0.125, dtype)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_split_plan_on_a_tail_past_half_the_slots(dtype):
    """One head, 300 work items of 256 query rows, 2048 keys: on 2 x 256
    slots the whole launch is a tail past half the slots, which the plan
    cuts into 3 key ranges of 10-11 blocks (900 parts in two rounds of a
    third; no test hook).  Sampled query rows of several items against
    fp64."""
    rng = np.random.default_rng(22)
    sq, sk = 300 * 256, 2048
    q = rnd(rng, (1, sq, 64), 1.0, dtype)
    k = rnd(rng, (1, sk, 64), 1.0, dtype)
    v = rnd(rng, (1, sk, 64), 1.0, dtype)
    g = cu()
    o = down(g.dev_scaled_dot_product_attention(up(q, dtype), up(k, dtype), up(v, dtype), 0.125))
    rows = np.unique(np.r_[0, 255, 256, sq // 2, sq // 2 + 129, sq - 257, sq - 1,
                           np.random.default_rng(3).choice(sq, 120, replace=False)])
    ref = sdpa64(q[:, rows], k, v, 0.125)
    assert float(np.max(np.abs(o[:, rows] - ref))) <= bound(q, k, v, 0.125, dtype)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("sk", [65, 100, 177, 4095])
def test_rows_past_sk_are_never_read(dtype, sk):
    """Keys and values past Sk inside the same allocation hold NaN: the
    last, partial key block must read them as zeros (the buffer bound of
    Sk rows), so the output stays finite and matches fp64.  Two batch
    entries, each followed by 64 NaN rows, so entry 0's tail lies inside
    entry 1's stride."""
    b, sq, pad = 2, 130, 64
    rng = np.random.default_rng(sk)
    q = rnd(rng, (b, sq, 64), 1.0, dtype)
    k = rnd(rng, (b, sk, 64), 1.0, dtype)
    v = rnd(rng, (b, sk, 64), 1.0, dtype)
    kp = np.full((b, sk + pad, 64), np.nan, np.float32)
    vp = np.full((b, sk + pad, 64), np.nan, np.float32)
    kp[:, :sk], vp[:, :sk] = k, v
    g = cu()
    gq, gk, gv = up(q, dtype), up(kp, dtype), up(vp, dtype)
    go = up(np.zeros((b, sq, 64), np.float32), dtype)
    so = ctypes.CDLL(os.path.join(ROOT, "scaffolding_amd", "libsfgemm.so"))
    so.sf_last_error.restype = ctypes.c_char_p
    I64, P = ctypes.c_int64, ctypes.c_void_p
    st = (sk + pad) * 64
    rc = so.sf_attention(P(gq.data_ptr), I64(64), I64(sq * 64), P(gk.data_ptr), I64(64), I64(st),
                         P(gv.data_ptr), I64(64), I64(st), P(go.data_ptr), I64(64), I64(sq * 64),
                         I64(b), I64(sq), I64(sk), I64(64), ctypes.c_float(0.125), 2 if dtype == "bfloat16" else 1,
                         None)
    assert rc == 0, so.sf_last_error()
    g.device_synchronize()
    o = down(go)
    assert np.all(np.isfinite(o))
    o64 = sdpa64(q, k, v, 0.125)
    assert float(np.max(np.abs(o - o64))) <= bound(q, k, v, 0.125, dtype)
