"""Writes the committed golden fixtures of the oracle tests.

The reference holds no golden vectors for this path (its only GEMM
known-answer test is the macOS Accelerate check tests/test_mps_ops.py:24-41,
which compares against NumPy at runtime), so these fixtures are computed
here independently of NumPy's BLAS:

  tiny_gemm.npz        ragged tiny GEMMs (NN and NT, each input dtype) with
                       C computed by Python triple loops in math.fsum
                       (exactly rounded sums of fp64 products)
  tiny_linear.npz      tiny linear layers with bias and SiLU / GELU-tanh
                       epilogues evaluated with the math module, per element
  tiny_backward.npz    tiny linear-layer gradients (grad_input = g W,
                       grad_weight = g^T x, grad_bias = column sums of g)
                       by triple loops / column loops in math.fsum
  tiny_norm.npz        tiny layer norms (with gamma, beta and a per-row
                       adaptive scale / shift) and RMS norms, row by row in
                       math.fsum, and tiny single-head attentions (ragged
                       key counts) with fsum dot products and softmax sums
  tiny_mask.npz        tiny attentions with an additive mask (reference
                       nn/functional.py:339-341: scores * scale + mask,
                       NumPy broadcasting, -inf entries) per row in fsum
  tiny_dit.npz         one tiny DiT block (self-attention, cross-attention
                       and the SiLU MLP, reference diffusion/models.py:538-590)
                       evaluated in pure Python lists with math.fsum: every
                       linear, norm, head split, softmax and residual
  config_inputs.json   shape, dtype and SHA-256 of every generated input of
                       BASELINE.json's five configs (oracle.configs), so the
                       generators are pinned across machines

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import configs as cfg  # noqa: E402
from oracle.quant import quantize  # noqa: E402

TINY_SHAPES = [(1, 1, 1), (3, 5, 7), (4, 3, 2), (2, 9, 16), (5, 4, 33), (7, 6, 24)]
DTYPES = ["float32", "float16", "bfloat16"]


def fsum_matmul(a, b):
    m, k = a.shape
    n = b.shape[1]
    out = np.empty((m, n), np.float64)
    for i in range(m):
        for j in range(n):
            out[i, j] = math.fsum(float(a[i, p]) * float(b[p, j]) for p in range(k))
    return out


def silu(v):
    return v / (1.0 + math.exp(-v)) if v > -700 else 0.0


def gelu(v):
    return 0.5 * v * (1.0 + math.tanh(math.sqrt(2.0 / math.pi) * (v + 0.044715 * v ** 3)))


def tiny_gemm():
    rng = np.random.default_rng(20261201)
    arrays = {}
    for dt in DTYPES:
        for (m, n, k) in TINY_SHAPES:
            a = quantize(rng.uniform(-2, 2, (m, k)).astype(np.float32), dt)
            b = quantize(rng.uniform(-2, 2, (k, n)).astype(np.float32), dt)
            key = "%s_%dx%dx%d" % (dt, m, n, k)
            arrays[key + "_a"] = a
            arrays[key + "_b"] = b             # K x N
            arrays[key + "_c"] = fsum_matmul(a, b)
    np.savez(os.path.join(HERE, "tiny_gemm.npz"), **arrays)


def tiny_linear():
    rng = np.random.default_rng(7)
    arrays = {}
    for dt in DTYPES:
        for (m, n, k) in [(3, 5, 7), (2, 4, 16)]:
            x = quantize(rng.uniform(-3, 3, (m, k)).astype(np.float32), dt)
            w = quantize(rng.uniform(-1, 1, (n, k)).astype(np.float32), dt)
            b = quantize(rng.uniform(-1, 1, (n,)).astype(np.float32), dt)
            pre = fsum_matmul(x, w.T) + b.astype(np.float64)
            key = "%s_%dx%dx%d" % (dt, m, n, k)
            arrays[key + "_x"] = x
            arrays[key + "_w"] = w
            arrays[key + "_b"] = b
            arrays[key + "_bias"] = pre
            arrays[key + "_silu"] = np.vectorize(silu)(pre)
            arrays[key + "_gelu"] = np.vectorize(gelu)(pre)
    np.savez(os.path.join(HERE, "tiny_linear.npz"), **arrays)


def tiny_backward():
    rng = np.random.default_rng(793)
    arrays = {}
    for dt in DTYPES:
        for (m, n, k) in [(1, 3, 2), (5, 4, 7), (9, 6, 16), (3, 8, 5)]:
            g = quantize(rng.uniform(-2, 2, (m, n)).astype(np.float32), dt)
            x = quantize(rng.uniform(-2, 2, (m, k)).astype(np.float32), dt)
            w = quantize(rng.uniform(-1, 1, (n, k)).astype(np.float32), dt)
            key = "%s_%dx%dx%d" % (dt, m, n, k)
            arrays[key + "_g"] = g
            arrays[key + "_x"] = x
            arrays[key + "_w"] = w
            arrays[key + "_dx"] = fsum_matmul(g, w)
            gt = np.ascontiguousarray(g.T)
            arrays[key + "_dw"] = fsum_matmul(gt, x)
            arrays[key + "_db"] = np.array([math.fsum(float(g[i, j]) for i in range(m)) for j in range(n)])
    np.savez(os.path.join(HERE, "tiny_backward.npz"), **arrays)


def lnorm_rows(x, gamma, beta, eps, ms=None, mt=None):
    out = []
    for r, row in enumerate(x):
        n = len(row)
        mu = math.fsum(row) / n
        var = math.fsum((v - mu) ** 2 for v in row) / n
        rs = 1.0 / math.sqrt(var + eps)
        y = []
        for j, v in enumerate(row):
            h = (v - mu) * rs * gamma[j] + beta[j]
            if ms is not None:
                h = h * (1.0 + ms[r][j]) + mt[r][j]
            y.append(h)
        out.append(y)
    return out


def attn_rows(q, k, v, scale):
    out = []
    for qi in q:
        s = [scale * math.fsum(a * b for a, b in zip(qi, kj)) for kj in k]
        m = max(s)
        e = [math.exp(t - m) for t in s]
        z = math.fsum(e)
        out.append([math.fsum(e[j] * v[j][d] for j in range(len(k))) / z for d in range(len(v[0]))])
    return out


def tiny_norm():
    rng = np.random.default_rng(512)
    arrays = {}
    for (r, c) in [(1, 1), (3, 5), (4, 16), (2, 37)]:
        x = rng.uniform(-3, 3, (r, c)) + rng.uniform(-2, 2, (r, 1))
        g = rng.uniform(0.5, 1.5, c)
        b = rng.uniform(-0.5, 0.5, c)
        ms = rng.uniform(-0.5, 0.5, (r, c))
        mt = rng.uniform(-0.5, 0.5, (r, c))
        key = "ln_%dx%d" % (r, c)
        arrays[key + "_x"], arrays[key + "_g"], arrays[key + "_b"] = x, g, b
        arrays[key + "_ms"], arrays[key + "_mt"] = ms, mt
        xl = x.tolist()
        arrays[key + "_y"] = np.array(lnorm_rows(xl, g.tolist(), b.tolist(), 1e-5))
        arrays[key + "_ymod"] = np.array(lnorm_rows(xl, g.tolist(), b.tolist(), 1e-5, ms.tolist(), mt.tolist()))
        rms = []
        for row in xl:
            den = math.sqrt(math.fsum(v * v for v in row) / len(row) + 1e-6)
            rms.append([v / den * g[j] for j, v in enumerate(row)])
        arrays["rms_%dx%d_y" % (r, c)] = np.array(rms)
    for (n, s, d) in [(1, 1, 4), (3, 5, 8), (4, 67, 8)]:
        q = rng.uniform(-1, 1, (n, d))
        k = rng.uniform(-1, 1, (s, d))
        v = rng.uniform(-1, 1, (s, d))
        key = "attn_%dx%dx%d" % (n, s, d)
        arrays[key + "_q"], arrays[key + "_k"], arrays[key + "_v"] = q, k, v
        arrays[key + "_o"] = np.array(attn_rows(q.tolist(), k.tolist(), v.tolist(), 1.0 / math.sqrt(d)))
    np.savez(os.path.join(HERE, "tiny_norm.npz"), **arrays)


def tiny_mask():
    """Masked attention over [B, H, Sq, Sk] = [2, 3, 4, 6] scores, d = 8,
    with masks of four broadcast shapes; some entries -inf (never a whole
    row).  Each output row: s_j = scale * fsum(q . k_j) + mask_j, then the
    max-shifted exponentials and their fsum, per element."""
    rng = np.random.default_rng(339)
    b, h, sq, sk, d = 2, 3, 4, 6, 8
    scale = 1.0 / math.sqrt(d)
    arrays = {}
    for name, mshape in [("qk", (sq, sk)), ("b1qk", (b, 1, sq, sk)), ("bh1k", (b, h, 1, sk)), ("1k", (1, sk))]:
        q = rng.uniform(-2, 2, (b, h, sq, d))
        k = rng.uniform(-2, 2, (b, h, sk, d))
        v = rng.uniform(-1, 1, (b, h, sk, d))
        mask = rng.uniform(-3, 3, mshape)
        flat = mask.reshape(-1)
        flat[rng.choice(flat.size, size=max(1, flat.size // 6), replace=False)] = -np.inf
        # no row may be masked completely (that row would be NaN)
        full = np.broadcast_to(mask, (b, h, sq, sk))
        assert np.all(np.isfinite(full).any(axis=-1))
        o = np.empty((b, h, sq, d))
        for bi in range(b):
            for hi in range(h):
                for i in range(sq):
                    qi = q[bi, hi, i].tolist()
                    s = [scale * math.fsum(x * y for x, y in zip(qi, k[bi, hi, j].tolist())) + float(full[bi, hi, i, j])
                         for j in range(sk)]
                    m = max(s)
                    e = [math.exp(t - m) for t in s]
                    z = math.fsum(e)
                    for dd in range(d):
                        o[bi, hi, i, dd] = math.fsum(e[j] * float(v[bi, hi, j, dd]) for j in range(sk)) / z
        key = "mask_" + name
        arrays[key + "_q"], arrays[key + "_k"], arrays[key + "_v"] = q, k, v
        arrays[key + "_mask"], arrays[key + "_o"] = mask, o
    np.savez(os.path.join(HERE, "tiny_mask.npz"), **arrays)


def tiny_dit():
    """B = 1, N = 3 tokens, C = 4 (2 heads of 2), cond_dim 3, context of 2
    tokens of width 5, MLP hidden 16."""
    rng = np.random.default_rng(538)
    N, C, H, CD, S, XD = 3, 4, 2, 3, 2, 5
    D = C // H
    p = {}

    def lin(name, i, o, bias=True):
        p[name + ".weight"] = rng.uniform(-0.6, 0.6, (o, i))
        if bias:
            p[name + ".bias"] = rng.uniform(-0.2, 0.2, o)

    for nm in ("norm1", "norm2", "norm3"):
        p[nm + ".norm.weight"] = rng.uniform(0.7, 1.3, C)
        p[nm + ".norm.bias"] = rng.uniform(-0.2, 0.2, C)
        lin(nm + ".linear", CD, 2 * C)
    lin("to_qkv", C, 3 * C, bias=False)
    lin("self_out", C, C)
    lin("cross_q", C, C, bias=False)
    lin("cross_k", XD, C, bias=False)
    lin("cross_v", XD, C, bias=False)
    lin("cross_out", C, C)
    lin("ff.0", C, 4 * C)
    lin("ff.3", 4 * C, C)
    x = rng.uniform(-2, 2, (1, N, C))
    cond = rng.uniform(-1, 1, (1, CD))
    ctx = rng.uniform(-1, 1, (1, S, XD))

    L = {k: v.tolist() for k, v in p.items()}

    def linear(rows, name, act=None):
        w = L[name + ".weight"]
        b = L.get(name + ".bias")
        out = []
        for r in rows:
            y = []
            for j, wj in enumerate(w):
                t = math.fsum(a * c for a, c in zip(r, wj)) + (b[j] if b is not None else 0.0)
                y.append(t / (1.0 + math.exp(-t)) if act == "silu" else t)
            out.append(y)
        return out

    def ada(rows, nm):
        prm = linear(cond.tolist(), nm + ".linear")[0]
        ms = [prm[:C]] * len(rows)
        mt = [prm[C:]] * len(rows)
        return lnorm_rows(rows, L[nm + ".norm.weight"], L[nm + ".norm.bias"], 1e-5, ms, mt)

    def mha(qr, kr, vr):
        out = [[0.0] * C for _ in qr]
        for h in range(H):
            sl = slice(h * D, (h + 1) * D)
            o = attn_rows([r[sl] for r in qr], [r[sl] for r in kr], [r[sl] for r in vr], 1.0 / math.sqrt(D))
            for i, row in enumerate(o):
                out[i][sl] = row
        return out

    xr = x[0].tolist()
    h = ada(xr, "norm1")
    qkv = linear(h, "to_qkv")
    sa = mha([r[:C] for r in qkv], [r[C:2 * C] for r in qkv], [r[2 * C:] for r in qkv])
    so = linear(sa, "self_out")
    xr = [[a + b for a, b in zip(r1, r2)] for r1, r2 in zip(xr, so)]
    x_sa = [list(r) for r in xr]
    h2 = ada(xr, "norm2")
    ca = mha(linear(h2, "cross_q"), linear(ctx[0].tolist(), "cross_k"), linear(ctx[0].tolist(), "cross_v"))
    co = linear(ca, "cross_out")
    xr = [[a + b for a, b in zip(r1, r2)] for r1, r2 in zip(xr, co)]
    f = linear(ada(xr, "norm3"), "ff.0", "silu")
    fo = linear(f, "ff.3")
    y_cross = [[a + b for a, b in zip(r1, r2)] for r1, r2 in zip(xr, fo)]
    # without the context: FFN straight after self-attention
    f = linear(ada(x_sa, "norm3"), "ff.0", "silu")
    fo = linear(f, "ff.3")
    y_self = [[a + b for a, b in zip(r1, r2)] for r1, r2 in zip(x_sa, fo)]
    arrays = {"p_" + k: v for k, v in p.items()}
    arrays.update(x=x, cond=cond, context=ctx, heads=np.array(H), y_self=np.array([y_self]),
                  y_cross=np.array([y_cross]))
    np.savez(os.path.join(HERE, "tiny_dit.npz"), **arrays)


def digest(a: np.ndarray) -> dict:
    a = np.ascontiguousarray(a, dtype=np.float32)
    return {"shape": list(a.shape), "sha256": hashlib.sha256(a.tobytes()).hexdigest(),
            "first": [float(v) for v in a.reshape(-1)[:4]]}


def config_inputs():
    out = {}
    c1 = cfg.c1_linear()
    out["C1"] = {"x": digest(c1.x), "w": digest(c1.w), "b": digest(c1.b)}
    a, b = cfg.c2_matmul(1024)
    out["C2_1024"] = {"a": digest(a), "b": digest(b)}
    for m in (1, 16):
        c3 = cfg.c3_linear(m)
        out["C3_M%d" % m] = {"x": digest(c3.x), "w": digest(c3.w), "b": digest(c3.b)}
    q, k, v, _ = cfg.c4_attention()
    out["C4"] = {"q": digest(q), "k": digest(k), "v": digest(v)}
    c5 = cfg.c5_projection("out")
    out["C5_out"] = {"x": digest(c5.x), "w": digest(c5.w), "b": digest(c5.b)}
    with open(os.path.join(HERE, "config_inputs.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    # python tests/golden/make_golden.py [fixture ...]: all, or the named ones
    makers = {"tiny_gemm": tiny_gemm, "tiny_linear": tiny_linear, "tiny_backward": tiny_backward,
              "tiny_norm": tiny_norm, "tiny_mask": tiny_mask, "tiny_dit": tiny_dit, "config_inputs": config_inputs}
    for name in sys.argv[1:] or list(makers):
        makers[name]()
    print("fixtures written to", HERE)
