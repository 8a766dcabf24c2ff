#!/usr/bin/env python3
"""Benchmark of the matmul hot path on one MI355X.

Headline (``value``): the north-star workload of BASELINE.json — bf16
``linear_forward`` (GEMM + bias epilogue, fp32 accumulate) at
M = N = K = 4096 — in TFLOP/s.  A "step" is one ``dev_linear_forward``
launch over one resident 4096 x 4096 activation; K steps are timed with HIP
events on the launch stream, bracketed by device synchronisation.  Every
warm-up runs at least W steps and at least SETTLE_MS of device work: after
idle the chip spends its first ~30 ms of load at a lower clock, so a short
warm-up would time that transient instead of the sustained rate.  The JSON
line reports the warm-up as run and the rate of its first steps.

``sweep`` times every other config of BASELINE.json the same way (C1 fp32
Linear, C2 fp32 square matmul, C3 bf16 Linear+bias+SiLU at M = 1 / 16 /
4096, C4 fp16 attention QK^T / softmax / PV, C5 bf16 DiT projections, their
backward GEMMs, and the DiT block glue at C5's shape), with
TFLOP/s or HBM GB/s and the roofline fraction.  HBM-bound skinny rows rotate
four weight copies (> the 256 MB Infinity Cache) across steps.

``cpu_baseline`` times the reference's Linux CPU path for the headline
workload (NumPy fp32 ``x @ W.T + b``, reference nn/layers.py:129-131) on the
host's BLAS threads, GC off, 1 warm-up, median of a bounded sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-sweep]
                       [--no-cpu] [--only NAME]
"""
from __future__ import annotations

import argparse
import gc
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GEMM TFLOP/s & % MFMA peak (bf16/fp32 linear); skinny GEMM HBM GB/s"
PEAK_BF16 = 2.5e15      # dense bf16/fp16 MFMA, FLOP/s
PEAK_FP32 = 157.3e12    # fp32 matrix, FLOP/s
PEAK_HBM = 8.0e12       # HBM3E, B/s
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_gemm16nt_4w_linear_4096.txt")
SETTLE_MS = 100.0       # minimum device work in every warm-up (see Dev.time_steps)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Dev:
    """Synthetic resident inputs and event timing on the default stream."""

    def __init__(self):
        import scaffolding_amd as sf
        self.sf = sf
        self.cu = sf._cuops
        self.rng = np.random.default_rng(1234)

    def rand(self, shape, std, dtype):
        # Host float32 normal draws, rounded to `dtype` by the device cast.
        a = (self.rng.standard_normal(shape, dtype=np.float32) * np.float32(std))
        return self.cu.gputensor_from_numpy(a, 0, dtype)

    def time_steps(self, fn, steps, warmup, info=None):
        """Mean ms per call of fn over `steps` calls enqueued back to back
        between two events, after the warm-up: at least `warmup` calls and
        at least SETTLE_MS of device work.  The chip needs that long under
        load to leave its power-management transient (measured: the first
        ~100 launches of the 4096^3 GEMM after idle take 0.110 ms, then the
        clock recovers and holds 0.0965 ms for thousands of launches), so
        the timed region measures the sustained rate.  `info` (a dict)
        receives the warm-up's own figures, the transient included."""
        cu = self.cu
        keep = []

        def call(i):
            keep.append(fn(i))
            if len(keep) > 8:
                keep.pop(0)
        # The warm-up keeps the same window of live outputs as the timed
        # loop, so the caching allocator already holds every block the timed
        # loop needs (no device allocation inside the timed region).
        n0 = max(warmup, 9)
        w0, w1 = cu.CudaEvent(), cu.CudaEvent()
        cu.device_synchronize()
        w0.record()
        for i in range(n0):
            call(i)
        w1.record()
        w1.synchronize()
        first_ms = w0.elapsed_time(w1)
        # More warm-up in chunks of about 20 ms of device work, each sized
        # from the rate of the chunk before, until SETTLE_MS have run.
        per = max(first_ms / n0, 1e-3)
        settle_ms, extra = 0.0, 0
        while first_ms + settle_ms < SETTLE_MS:
            chunk = max(1, min(int(np.ceil((SETTLE_MS - first_ms - settle_ms) / per)), int(20.0 / per) + 1))
            w0.record()
            for i in range(chunk):
                call(n0 + extra + i)
            w1.record()
            w1.synchronize()
            t = w0.elapsed_time(w1)
            settle_ms += t
            extra += chunk
            per = max(t / chunk, 1e-3)
        if info is not None:
            info.update({"warmup_steps_run": n0 + extra, "warmup_ms": round(first_ms + settle_ms, 2),
                         "first_steps": n0, "first_ms_per_step": round(first_ms / n0, 5)})
        e0, e1 = cu.CudaEvent(), cu.CudaEvent()
        e0.record()
        e0.synchronize()
        gc.disable()
        try:
            # A few untimed calls queue work ahead of the start event, so the
            # GPU is busy when it records and host-side launch latency does
            # not open an idle gap inside the timed region.
            for i in range(4):
                call(i)
            e0.record()
            for i in range(steps):
                call(i)
            e1.record()
            e1.synchronize()
        finally:
            gc.enable()
        cu.device_synchronize()
        return e0.elapsed_time(e1) / steps


def headline(d: Dev, steps: int, warmup: int):
    cu = d.cu
    m = n = k = 4096
    x = d.rand((m, k), 1.0, "bfloat16")
    w = d.rand((n, k), 0.02, "bfloat16")
    b = d.rand((n,), 0.01, "bfloat16")
    kern = cu.gemm_plan(1, m, n, k, 1, x.data_ptr, k, 0, w.data_ptr, k, 0, n, 0, x.dtype,
                        epi=1, ptr_bias=b.data_ptr)
    info = {}
    ms = d.time_steps(lambda i: cu.dev_linear_forward(x, w, b), steps, warmup, info)
    flops = 2.0 * m * n * k
    return {"ms": ms, "flops": flops, "kernel": kern, "m": m, "n": n, "k": k, "warmup_info": info,
            "bytes": float((m * k + n * k + m * n) * 2 + n * 2)}


def sweep(d: Dev, steps: int, warmup: int, only: str | None):
    cu = d.cu
    out = {}

    def want(name):
        return only is None or only in name

    def rec(name, ms, flops, nbytes, bound, peak_flops):
        t = ms * 1e-3
        tf = flops / t
        bw = nbytes / t
        r = {"ms": round(ms, 5), "tflops": round(tf / 1e12, 2), "gbps": round(bw / 1e9, 1)}
        if bound == "hbm":
            r["roofline"] = {"bound": "hbm", "frac": round(bw / PEAK_HBM, 4)}
        else:
            r["roofline"] = {"bound": "mfma", "frac": round(tf / peak_flops, 4)}
        out[name] = r
        log("  %-34s %9.4f ms  %8.2f TFLOP/s  %8.1f GB/s  %s %.1f%%" % (
            name, ms, tf / 1e12, bw / 1e9, bound, 100 * r["roofline"]["frac"]))

    # C1: fp32 nn.Linear 64x512 -> 512 (+b); launch-latency bound, report time.
    if want("C1"):
        x = d.rand((64, 512), 1.0 / np.sqrt(512), np.float32)
        w = d.rand((512, 512), 1.0 / np.sqrt(512), np.float32)
        b = d.rand((512,), 0.05, np.float32)
        ms = d.time_steps(lambda i: cu.dev_linear_forward(x, w, b), steps * 4, warmup)
        rec("C1_fp32_linear_64x512x512", ms, 2.0 * 64 * 512 * 512,
            (64 * 512 + 512 * 512 + 64 * 512 + 512) * 4.0, "mfma", PEAK_FP32)

    # C2: fp32 square matmul.
    for nn_ in (1024, 2048, 4096):
        if not want("C2_fp32_matmul_%d" % nn_):
            continue
        a = d.rand((nn_, nn_), 0.5, np.float32)
        bb = d.rand((nn_, nn_), 0.5, np.float32)
        ms = d.time_steps(lambda i: cu.dev_matmul(a, bb), max(5, steps // (nn_ // 1024)), warmup)
        rec("C2_fp32_matmul_%d" % nn_, ms, 2.0 * nn_ ** 3, 3.0 * nn_ * nn_ * 4, "mfma", PEAK_FP32)

    # C3: bf16 Linear + bias + SiLU, K 4096 -> N 11008.
    for m in (1, 16, 4096):
        name = "C3_bf16_linear_silu_M%d" % m
        if not want(name):
            continue
        k, n = 4096, 11008
        x = d.rand((m, k), 1.0, "bfloat16")
        copies = 4 if m <= 16 else 1
        ws = [d.rand((n, k), 0.02, "bfloat16") for _ in range(copies)]
        b = d.rand((n,), 0.01, "bfloat16")
        ms = d.time_steps(lambda i: cu.dev_linear_forward(x, ws[i % copies], b, "silu"), steps, warmup)
        nbytes = (m * k + n * k + m * n) * 2.0 + n * 2
        rec(name, ms, 2.0 * m * n * k, nbytes, "hbm" if m <= 16 else "mfma", PEAK_BF16)
        del ws

    # C4: fp16 attention, 60 heads x 4096 x 64.
    c4 = ["C4_fp16_qkT_scaled", "C4_fp16_softmax", "C4_fp16_pv", "C4_fp16_sdpa_3kernel", "C4_fp16_sdpa_fused"]
    if any(want(n) for n in c4):
        bh, s, dd = 60, 4096, 64
        q = d.rand((bh, s, dd), 1.0, np.float16)
        kk = d.rand((bh, s, dd), 1.0, np.float16)
        v = d.rand((bh, s, dd), 1.0, np.float16)
        st = max(3, steps // 10)
        if want("C4_fp16_qkT_scaled"):
            ms = d.time_steps(lambda i: cu.dev_batched_matmul_nt(q, kk, 0.125), st, 2)
            rec("C4_fp16_qkT_scaled", ms, 2.0 * bh * s * s * dd, bh * (2 * s * dd + s * s) * 2.0, "hbm", PEAK_BF16)
        if want("C4_fp16_softmax") or want("C4_fp16_pv"):
            scores = cu.dev_batched_matmul_nt(q, kk, 0.125)
            if want("C4_fp16_softmax"):
                ms = d.time_steps(lambda i: cu.dev_softmax(scores, -1), st, 2)
                rec("C4_fp16_softmax", ms, 0.0, bh * s * s * 2 * 2.0, "hbm", PEAK_BF16)
            probs = cu.dev_softmax(scores, -1)
            del scores
            if want("C4_fp16_pv"):
                ms = d.time_steps(lambda i: cu.dev_batched_matmul(probs, v), st, 2)
                rec("C4_fp16_pv", ms, 2.0 * bh * s * s * dd, bh * (s * s + 2 * s * dd) * 2.0, "hbm", PEAK_BF16)
            del probs
        if want("C4_fp16_sdpa_3kernel"):
            ms = d.time_steps(lambda i: cu.dev_sdpa_unfused(q, kk, v, 0.125), st, 1)
            rec("C4_fp16_sdpa_3kernel", ms, 4.0 * bh * s * s * dd, bh * (4 * s * dd + 4 * s * s) * 2.0, "hbm",
                PEAK_BF16)
        if want("C4_fp16_sdpa_fused"):
            # One fused launch (sf_attention): compute-bound, 4 * S^2 * D flop per head.
            ms = d.time_steps(lambda i: cu.dev_scaled_dot_product_attention(q, kk, v, 0.125), max(5, steps // 2), 2)
            rec("C4_fp16_sdpa_fused", ms, 4.0 * bh * s * s * dd, bh * 4 * s * dd * 2.0, "mfma", PEAK_BF16)

    # C5: bf16 DiT projections, 17776 tokens.
    tokens = 13 * (60 * 90 // 4) + 226
    for pname, (k, n, has_b, act) in {"qkv": (1920, 5760, False, None), "out": (1920, 1920, True, None),
                                      "mlp_up": (1920, 7680, True, "gelu"),
                                      "mlp_down": (7680, 1920, True, None)}.items():
        name = "C5_bf16_%s" % pname
        if not want(name):
            continue
        x = d.rand((tokens, k), 1.0, "bfloat16")
        w = d.rand((n, k), 0.02, "bfloat16")
        b = d.rand((n,), 0.01, "bfloat16") if has_b else None
        ms = d.time_steps(lambda i: cu.dev_linear_forward(x, w, b, act), steps, warmup)
        rec(name, ms, 2.0 * tokens * n * k, (tokens * k + n * k + tokens * n) * 2.0, "mfma", PEAK_BF16)
        del x, w

    # C5 training step's backward GEMMs (next on the path after the forward):
    # dX = dY W (NN), dW = dY^T X (TN over the 17776 tokens), db = column
    # sums of dY, one dev_linear_backward call.  Work: 4 * tokens * N * K.
    for pname, (k, n, has_b) in {"qkv": (1920, 5760, False), "out": (1920, 1920, True),
                                 "mlp_up": (1920, 7680, True), "mlp_down": (7680, 1920, True)}.items():
        name = "C5bwd_bf16_%s" % pname
        if not want(name):
            continue
        x = d.rand((tokens, k), 1.0, "bfloat16")
        w = d.rand((n, k), 0.02, "bfloat16")
        g = d.rand((tokens, n), 1.0, "bfloat16")
        ms = d.time_steps(lambda i: cu.dev_linear_backward(g, x, w, has_b), max(5, steps // 2), warmup)
        rec(name, ms, 4.0 * tokens * n * k, (2 * tokens * n + 2 * tokens * k + 2 * n * k) * 2.0, "mfma", PEAK_BF16)
        del x, w, g

    # C5 DiT block glue at the same shape: the fused adaptive layer norm, the
    # fused attention over the 30 packed heads (17776 x 17776 per head), and
    # the whole GPU-resident DiTBlock forward (reference
    # diffusion/models.py:538-590, self-attention + SiLU MLP, cond_dim 512).
    if want("C5_bf16_ada_layer_norm"):
        x = d.rand((1, tokens, 1920), 1.0, "bfloat16")
        prm = d.rand((1, 2 * 1920), 0.1, "bfloat16")
        gm = d.rand((1920,), 1.0, "bfloat16")
        bt = d.rand((1920,), 0.1, "bfloat16")
        ms = d.time_steps(lambda i: cu.dev_ada_layer_norm(x, prm, 1e-5, gm, bt), steps, warmup)
        rec("C5_bf16_ada_layer_norm", ms, 0.0, 2.0 * tokens * 1920 * 2, "hbm", PEAK_BF16)
        del x
    if want("C5_bf16_attention_packed"):
        qkv = d.rand((1, tokens, 3 * 1920), 1.0, "bfloat16")
        ms = d.time_steps(lambda i: cu.dev_attention_packed(qkv, 30), max(3, steps // 10), 2)
        rec("C5_bf16_attention_packed", ms, 4.0 * 30 * tokens * tokens * 64, 4.0 * tokens * 1920 * 2, "mfma",
            PEAK_BF16)
        del qkv
    if want("C5_bf16_dit_block"):
        import scaffolding_amd as sf
        from scaffolding_amd.diffusion import DiTBlock
        dim, heads, cdim = 1920, 30, 512
        blk = DiTBlock(dim, heads, cdim, dtype="bfloat16")
        x = sf.Tensor._wrap_gpu(d.rand((1, tokens, dim), 1.0, "bfloat16"))
        cond = sf.Tensor._wrap_gpu(d.rand((1, cdim), 1.0, "bfloat16"))
        ms = d.time_steps(lambda i: blk(x, cond)._gpu, max(3, steps // 10), 2)
        proj = 2.0 * tokens * dim * (3 * dim + dim + 4 * dim + 4 * dim) + 3 * 2.0 * cdim * 2 * dim
        rec("C5_bf16_dit_block", ms, proj + 4.0 * heads * tokens * tokens * (dim // heads),
            (tokens * dim * 2 * 11 + 12 * dim * dim) * 2.0, "mfma", PEAK_BF16)
        del blk, x

    # Headline variant with the SiLU epilogue fused.
    if want("north_star_bias_silu"):
        x = d.rand((4096, 4096), 1.0, "bfloat16")
        w = d.rand((4096, 4096), 0.02, "bfloat16")
        b = d.rand((4096,), 0.01, "bfloat16")
        ms = d.time_steps(lambda i: cu.dev_linear_forward(x, w, b, "silu"), steps, warmup)
        rec("north_star_bf16_linear_bias_silu_4096", ms, 2.0 * 4096 ** 3, 3 * 4096 * 4096 * 2.0, "mfma",
            PEAK_BF16)
    # HBM write probe, not a config: the library's zero fill (16-byte stores,
    # grid-stride) over 1 GiB, a write-only stream like the C4 score kernel's
    # 2 GB of output (the timing loop keeps 8 outputs live: 8 GiB, within
    # the caching allocator's limit, so no allocation in the timed region).
    if want("hbm_write_probe"):
        n1g = (1 << 30) // 4
        ms = d.time_steps(lambda i: cu.zeros((n1g,), np.float32, 0), max(5, steps // 4), warmup)
        rec("hbm_write_probe_zero_fill_1GiB", ms, 0.0, float(1 << 30), "hbm", PEAK_BF16)
    # Power probe, not a config: the headline GEMM (same kernel, same plan)
    # on constant operands (x = 1, W = 1/128, b = 0: every product and sum
    # is exact), whose multiplier inputs never toggle.  The gap to the
    # random-operand headline is what the chip's power limit takes.
    if want("power_probe"):
        m = n = k = 4096
        x = cu.gputensor_from_numpy(np.ones((m, k), np.float32), 0, "bfloat16")
        w = cu.gputensor_from_numpy(np.full((n, k), 1.0 / 128, np.float32), 0, "bfloat16")
        b = cu.gputensor_from_numpy(np.zeros((n,), np.float32), 0, "bfloat16")
        ms = d.time_steps(lambda i: cu.dev_linear_forward(x, w, b), steps, warmup)
        rec("power_probe_north_star_constant_operands", ms, 2.0 * m * n * k,
            float((m * k + n * k + m * n) * 2 + n * 2), "mfma", PEAK_BF16)
    return out


def cpu_baseline(budget_s: float = 20.0):
    """The reference CPU path for the headline workload, timed on the host."""
    from oracle import cpu_path  # the checker package; this leg only
    try:
        from threadpoolctl import threadpool_info
        threads = max([p.get("num_threads", 0) for p in threadpool_info()
                       if p.get("user_api") == "blas"] or [os.cpu_count() or 1])
    except Exception:  # noqa: BLE001
        threads = os.cpu_count() or 1
    rng = np.random.default_rng(7)
    m = n = k = 4096
    # bf16 inputs run as fp32 on the reference CPU path (reference dtype.py:31).
    x = rng.standard_normal((m, k), dtype=np.float32)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    b = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.01))
    gc.disable()
    try:
        t0 = time.perf_counter()
        cpu_path.linear(x, w, b)  # warm-up
        first = time.perf_counter() - t0
        trials = int(max(3, min(20, budget_s / max(first, 1e-3))))
        times = []
        for _ in range(trials):
            t0 = time.perf_counter()
            cpu_path.linear(x, w, b)
            times.append(time.perf_counter() - t0)
    finally:
        gc.enable()
    med = statistics.median(times)
    one = None
    try:  # the same workload on one BLAS thread, a few trials
        from threadpoolctl import threadpool_limits
        with threadpool_limits(limits=1, user_api="blas"):
            gc.disable()
            try:
                t1 = []
                for _ in range(3):
                    t0 = time.perf_counter()
                    cpu_path.linear(x, w, b)
                    t1.append(time.perf_counter() - t0)
            finally:
                gc.enable()
        m1 = statistics.median(t1)
        one = {"value": round(2.0 * m * n * k / m1 / 1e12, 4), "unit": "TFLOP/s", "cores": 1,
               "ms_per_step": round(m1 * 1e3, 1), "trials": len(t1)}
    except Exception as e:  # noqa: BLE001
        one = {"error": str(e)}
    return {"value": round(2.0 * m * n * k / med / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": "reference CPU path (NumPy fp32 x @ W.T + b, nn/layers.py:129-131) at "
                      "4096x4096x4096, bf16 inputs as fp32 per dtype.py:31; median of %d trials after 1 "
                      "warm-up, GC off, %d BLAS threads; %.3f s/trial" % (trials, threads, med),
            "ms_per_step": round(med * 1e3, 2),
            "cpu_model": _cpu_model(), "blas": _blas_name(),
            "host_cpus": os.cpu_count(), "host_cpus_usable": _usable_cpus(),
            "single_thread": one}


def _usable_cpus():
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return None


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def _blas_name():
    try:
        from threadpoolctl import threadpool_info
        for p in threadpool_info():
            if p.get("user_api") == "blas":
                return "%s %s" % (p.get("internal_api"), p.get("version"))
    except Exception:  # noqa: BLE001
        pass
    return None


def read_traffic():
    """HBM bytes per launch of the headline kernel from the committed
    rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE, copy-kernel scaled)."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def trace_summary(path: str, last: int) -> None:
    """Markdown summary of a rocprofv3 kernel-trace CSV: per kernel, every
    dispatch, and for the most launched kernel also its last `last`
    dispatches (the timed region of a bench.py run, whose warm-up comes
    first)."""
    import csv
    rows = list(csv.DictReader(open(path)))
    per = {}
    for r in rows:
        name = r["Kernel_Name"]
        per.setdefault(name, []).append((int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    total = sum(e - b for v in per.values() for b, e in v)
    print("| kernel | calls | avg µs | min µs | max µs | total µs | % |\n|---|---|---|---|---|---|---|")
    for name, v in sorted(per.items(), key=lambda kv: -sum(e - b for b, e in kv[1])):
        d = [(e - b) / 1e3 for b, e in v]
        print("| `%s` | %d | %.2f | %.2f | %.2f | %.1f | %.2f |" % (
            name[:110], len(d), sum(d) / len(d), min(d), max(d), sum(d), 100.0 * sum(d) * 1e3 / total))
    name, v = max(per.items(), key=lambda kv: len(kv[1]))
    v.sort()
    d = [(e - b) / 1e3 for b, e in v[-last:]]
    print("\nlast %d dispatches of `%s`: avg %.2f µs, min %.2f, max %.2f" % (
        len(d), name[:110], sum(d) / len(d), min(d), max(d)))


def pmc_summary(path: str, kernel: str | None, last: int) -> None:
    """Markdown summary of a rocprofv3 --pmc counter-collection CSV: for the
    dispatches whose kernel name contains `kernel` (default: the most
    dispatched kernel), the mean of each counter over the last `last` of
    them, and derived figures where their counters are present:
      clock      GRBM_GUI_ACTIVE / 8 XCDs / dispatch duration (the GRBM
                 count is the sum over the 8 XCDs of gfx950)
      MFMA busy  SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x GRBM_GUI_ACTIVE / 8)
      co-exec    SQ_VALU_MFMA_COEXEC_CYCLES / SQ_VALU_MFMA_BUSY_CYCLES
      L2 hit     TCC_HIT / (TCC_HIT + TCC_MISS)
      L1->L2 latency  TCP_TCC_READ_REQ_LATENCY / TCP_TCC_READ_REQ (cycles)"""
    import csv
    disp = {}
    for r in csv.DictReader(open(path)):
        d = disp.setdefault(int(r["Dispatch_Id"]), {"name": r["Kernel_Name"]})
        d[r["Counter_Name"]] = float(r["Counter_Value"])
        d["dur_us"] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    names = {}
    for d in disp.values():
        names[d["name"]] = names.get(d["name"], 0) + 1
    if kernel is None:
        pick = max(names, key=names.get)
        sel = [disp[i] for i in sorted(disp) if disp[i]["name"] == pick]
    else:
        sel = [disp[i] for i in sorted(disp) if kernel in disp[i]["name"]]
    if not sel:
        print("no dispatch matches %r" % kernel)
        return
    sel = sel[-last:]
    keys = sorted(k for k in sel[0] if k != "name")
    mean = {k: sum(d[k] for d in sel) / len(sel) for k in keys}
    print("kernel `%s`, mean over its last %d dispatches\n" % (sel[-1]["name"][:110], len(sel)))
    print("| counter | mean per dispatch |\n|---|---|")
    for k in keys:
        print("| %s | %.6g |" % (k, mean[k]))
    der = []
    gui = mean.get("GRBM_GUI_ACTIVE")
    if gui:
        der.append(("clock (GHz)", gui / 8 / mean["dur_us"] / 1e3))
        if "SQ_VALU_MFMA_BUSY_CYCLES" in mean:
            der.append(("MFMA busy (fraction of SIMD cycles)", mean["SQ_VALU_MFMA_BUSY_CYCLES"] / 1024 / (gui / 8)))
    if mean.get("SQ_VALU_MFMA_BUSY_CYCLES") and "SQ_VALU_MFMA_COEXEC_CYCLES" in mean:
        der.append(("VALU co-executing with MFMA (fraction of MFMA-busy)",
                    mean["SQ_VALU_MFMA_COEXEC_CYCLES"] / mean["SQ_VALU_MFMA_BUSY_CYCLES"]))
    if "TCC_HIT" in mean and "TCC_MISS" in mean:
        der.append(("L2 hit rate", mean["TCC_HIT"] / max(1.0, mean["TCC_HIT"] + mean["TCC_MISS"])))
    if mean.get("TCP_TCC_READ_REQ") and "TCP_TCC_READ_REQ_LATENCY" in mean:
        der.append(("L1->L2 read latency (cycles)", mean["TCP_TCC_READ_REQ_LATENCY"] / mean["TCP_TCC_READ_REQ"]))
    if der:
        print("\n| derived | value |\n|---|---|")
        for k, v in der:
            print("| %s | %.4g |" % (k, v))


_TORCH_TIMER = r"""
import json, sys, time
import torch
import torch.nn.functional as tf
m, n, k, steps = (int(a) for a in sys.argv[1:5])
g = torch.Generator(device="cuda").manual_seed(7)
x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
w = (torch.randn((n, k), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
b = (torch.randn((n,), device="cuda", generator=g) * 0.01).to(torch.bfloat16)
res = []
for _ in range(3):
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.2:  # past the power transient
        for _ in range(10):
            tf.linear(x, w, b)
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        tf.linear(x, w, b)
    e1.record()
    e1.synchronize()
    res.append(e0.elapsed_time(e1) / steps)
print(json.dumps({"torch": torch.__version__, "ms": res}))
"""


def vendor_comparator(d: Dev, steps: int):
    """Comparator only, never on the product path: the same bf16 linear
    (x @ W^T + b) through PyTorch (torch.nn.functional.linear: hipBLASLt on
    ROCm, in a child process with its own HIP runtime) and through this
    library, each timed three times past the 100 ms power transient on the
    same box.  Shapes: the north star (4096^3) and the C5 QKV projection
    (17776 x 1920 -> 5760)."""
    import subprocess
    cu = d.cu
    out = {}
    for name, (m, n, k) in {"north_star_4096": (4096, 4096, 4096), "C5_qkv": (17776, 5760, 1920)}.items():
        r = subprocess.run([sys.executable, "-c", _TORCH_TIMER, str(m), str(n), str(k), str(steps)],
                           capture_output=True, text=True, timeout=600)
        if r.returncode != 0:
            raise RuntimeError("torch timer failed: " + r.stderr[-2000:])
        tj = json.loads(r.stdout.strip().splitlines()[-1])
        gx, gw, gb = d.rand((m, k), 1.0, "bfloat16"), d.rand((n, k), 0.02, "bfloat16"), d.rand((n,), 0.01, "bfloat16")
        sf_ms = [d.time_steps(lambda i: cu.dev_linear_forward(gx, gw, gb), steps, 10) for _ in range(3)]
        fl = 2.0 * m * n * k
        out[name] = {"m": m, "n": n, "k": k, "torch_linear_ms": [round(v, 5) for v in tj["ms"]],
                     "sf_linear_ms": [round(v, 5) for v in sf_ms],
                     "torch_best_tflops": round(fl / (min(tj["ms"]) * 1e-3) / 1e12, 1),
                     "sf_best_tflops": round(fl / (min(sf_ms) * 1e-3) / 1e12, 1), "torch": tj["torch"]}
        log(name, out[name])
        del gx, gw, gb
    return {"comparator": out}


# (label, stream A, stream B or -1): the stream numbers of sfp_issue
# (scaffolding_amd/probes/hw_probes.hip)
HW_ISSUE_CASES = [
    ("16 x mfma16x16x32 alone", 1, -1),
    ("8 x mfma32x32x16 alone (same flops)", 6, -1),
    ("64 x v_fma_f32 alone", 2, -1),
    ("32 x v_exp_f32 alone", 3, -1),
    ("64 x (v_cvt_pk_bf16_f32 + v_xor_b32) alone", 7, -1),
    ("64 x v_max3_f32 alone", 8, -1),
    ("mfma16 + fma, one wave (1 : 4)", 4, -1),
    ("mfma16 + exp, one wave (1 : 2)", 5, -1),
    ("mfma16 | mfma16", 1, 1),
    ("fma | fma", 2, 2),
    ("exp | exp", 3, 3),
    ("cvt | cvt", 7, 7),
    ("max3 | max3", 8, 8),
    ("fma | exp", 2, 3),
    ("mfma16 | fma", 1, 2),
    ("mfma16 | exp", 1, 3),
    ("mfma16 | cvt", 1, 7),
    ("mfma32 | fma", 6, 2),
    ("mfma32 | exp", 6, 3),
]


def hw_probes() -> int:
    """Runs the measurement kernels of libsfprobe.so (built by build.py from
    scaffolding_amd/probes/) and prints markdown tables: cycles per
    iteration of instruction streams alone and on a SIMD shared by two waves,
    MFMA-only throughput on random and constant bf16 operands, and the LDS
    read rate per CU."""
    import ctypes

    path = os.path.join(ROOT, "scaffolding_amd", "libsfprobe.so")
    if not os.path.exists(path):
        print("bench.py: %s is missing; run __graft_entry__.build() first" % path, file=sys.stderr)
        return 2
    lib = ctypes.CDLL(path)
    dbl = ctypes.c_double
    iters = 2000
    print("## Issue streams (shader cycles per iteration, mean over waves; one workgroup per CU)\n")
    print("| streams | waves per SIMD | A cycles/iter | B cycles/iter |")
    print("|---|---|---|---|")
    for label, a, b in HW_ISSUE_CASES:
        cyc = (dbl * 2)()
        rc = lib.sfp_issue(a, b, iters, cyc)
        if rc != 0:
            print("bench.py: sfp_issue(%d, %d) failed (%d)" % (a, b, rc), file=sys.stderr)
            return 1
        print("| %s | %d | %.0f | %s |" % (label, 1 if b < 0 else 2, cyc[0], "-" if b < 0 else "%.0f" % cyc[1]),
              flush=True)
    print("\n## MFMA only: the 4096^3 GEMM's 8.39 M v_mfma_f32_16x16x32_bf16 per launch\n")
    print("| operands | us per launch | TFLOP/s | % of 2.5 PF |")
    print("|---|---|---|---|")
    for random, label in ((1, "random bf16"), (0, "constant (x = 1, w = 1/128)")):
        us, fl = dbl(0.0), dbl(0.0)
        rc = lib.sfp_mfma_rate(random, 2000, 300, ctypes.byref(us), ctypes.byref(fl))
        if rc != 0:
            print("bench.py: sfp_mfma_rate failed (%d)" % rc, file=sys.stderr)
            return 1
        tf = fl.value / (us.value * 1e-6) / 1e12
        print("| %s | %.2f | %.1f | %.1f |" % (label, us.value, tf, 100 * tf * 1e12 / PEAK_BF16), flush=True)
    bpn = dbl(0.0)
    rc = lib.sfp_lds_read(20000, 20, ctypes.byref(bpn))
    if rc != 0:
        print("bench.py: sfp_lds_read failed (%d)" % rc, file=sys.stderr)
        return 1
    print("\n## LDS reads: ds_read_b128 only, 8 waves per CU\n")
    print("%.1f bytes per ns per CU" % bpn.value, flush=True)
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default=None, help="run only sweep entries containing this text")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run one fp32 x*1.0 pass over 1 GiB (reads 1 GiB, writes 1 GiB): the "
                         "known-traffic kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--no-headline", action="store_true")
    ap.add_argument("--vendor-torch-only", default=None, metavar="M,N,K",
                    help="time only torch.nn.functional.linear at M x N x K in this process (no library "
                         "loaded), so a profiler run on this command sees the vendor kernel (a comparator only)")
    ap.add_argument("--vendor-comparator", action="store_true",
                    help="time torch.nn.functional.linear (hipBLASLt) beside this library's linear at the "
                         "north-star and C5 QKV shapes, past the power transient, and exit (a comparator only)")
    ap.add_argument("--pmc-summary", default=None, metavar="CSV",
                    help="print a markdown summary of a rocprofv3 --pmc counter-collection CSV (the last --steps "
                         "dispatches of the kernel named by --kernel, default the most dispatched) and exit")
    ap.add_argument("--kernel", default=None, help="kernel-name substring for --pmc-summary")
    ap.add_argument("--trace-summary", default=None, metavar="CSV",
                    help="print a markdown summary of a rocprofv3 kernel-trace CSV (the last --steps "
                         "dispatches of the most launched kernel separately) and exit; no GPU use")
    ap.add_argument("--hw-probes", action="store_true",
                    help="run the hardware measurement kernels (libsfprobe.so: issue streams, MFMA-only rate on "
                         "random and constant operands, LDS read rate) and exit")
    args = ap.parse_args(argv)
    if args.hw_probes:
        return hw_probes()
    if args.trace_summary:
        trace_summary(args.trace_summary, args.steps)
        return 0
    if args.pmc_summary:
        pmc_summary(args.pmc_summary, args.kernel, args.steps)
        return 0
    if args.vendor_torch_only:
        m, n, k = (int(v) for v in args.vendor_torch_only.split(","))
        sys.argv = ["torch-timer", str(m), str(n), str(k), str(args.steps)]
        exec(compile(_TORCH_TIMER, "torch-timer", "exec"), {"__name__": "__torch_timer__"})
        return 0
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build runs on one GPU only (the matmul hot path's kernels at one "
              "GPU's share); --gpus %d is not supported" % max(args.gpus, world), file=sys.stderr)
        return 2

    d = Dev()
    cu = d.cu
    cu.set_device(0)
    props = cu.get_device_properties(0)
    log("device:", props)
    if args.copy_calibration:
        src = cu.zeros(((1 << 30) // 4,), np.float32, 0)
        cu.device_synchronize()
        y = cu.dev_muls(src, 1.0)
        cu.device_synchronize()
        del y, src
    if args.vendor_comparator:
        print(json.dumps(vendor_comparator(d, args.steps)), flush=True)
        return 0
    if args.no_headline:
        sw = sweep(d, args.steps, args.warmup, args.only)
        print(json.dumps({"sweep": sw}), flush=True)
        return 0
    h = headline(d, args.steps, args.warmup)
    tflops = h["flops"] / (h["ms"] * 1e-3) / 1e12
    log("headline: %s  %.4f ms  %.1f TFLOP/s  (%.1f%% of %.2f PF)" % (
        h["kernel"], h["ms"], tflops, 100 * tflops * 1e12 / PEAK_BF16, PEAK_BF16 / 1e15))
    sw = {} if args.no_sweep else sweep(d, args.steps, args.warmup, args.only)
    cpu = None if args.no_cpu else cpu_baseline()
    line = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(h["ms"], 5),
        # the warm-up as run: at least `warmup` steps and SETTLE_MS of device
        # work; first_ms_per_step is the rate of the first steps after idle
        "warmup_run": h["warmup_info"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "north-star bf16 linear_forward (GEMM + bias epilogue, fp32 accumulate) "
                               "M=N=K=4096, x~N(0,1), W~N(0,0.02), b~N(0,0.01)",
                   "M": h["m"], "N": h["n"], "K": h["k"], "epilogue": "bias",
                   "kernel": h["kernel"], "parallelism": "single-gpu"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16 / 1e12,
                     "unit": "TFLOP/s", "frac": round(tflops * 1e12 / PEAK_BF16, 4),
                     "traffic": read_traffic()},
        "cpu_baseline": cpu,
        "sweep": sw,
        "device": {"name": props.get("name"), "arch": props.get("arch"),
                   "cus": props.get("multi_processor_count")},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
