"""sf_gemm_noalloc (the entry point that allocates nothing: its split plans
take their workspace from a fixed per-device scratch array) against
sf_gemm on the same inputs: the same plans, so the outputs must be
bit-identical.  Two split calls in a row, the second on a smaller problem,
then fp32 split-K and an unsplit shape; each noalloc call runs twice, so
the counters the first call leaves behind are shown to be cleared.  In a
fresh process, split-plan calls leave the device's free memory and the
library's workspace unchanged; under HIP graph capture (after one
uncaptured call) the captured call replays bit-identically."""
from __future__ import annotations

import ctypes
import json
import os
import subprocess
import sys

import numpy as np
import pytest

from helpers import cu, rnd, up
from oracle import cpu_path as ref
from oracle.configs import tol_16

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
I64, P, F = ctypes.c_int64, ctypes.c_void_p, ctypes.c_float
DT = {"float32": 0, "float16": 1, "bfloat16": 2}


@pytest.fixture(scope="module")
def lib():
    so = ctypes.CDLL(os.path.join(ROOT, "scaffolding_amd", "libsfgemm.so"))
    so.sf_last_error.restype = ctypes.c_char_p
    return so


def _plan(lib, ta, tb, m, n, k, a, lda, b, ldb, c, dt):
    buf = ctypes.create_string_buffer(96)
    rc = lib.sf_gemm_plan(ta, tb, I64(m), I64(n), I64(k), I64(1), P(a.data_ptr), I64(lda), I64(0), P(b.data_ptr),
                          I64(ldb), I64(0), P(c.data_ptr), I64(n), I64(0), DT[dt], DT[dt], F(1.0), None, 0, buf, 96)
    assert rc == 0, lib.sf_last_error()
    return buf.value.decode()


def _call(lib, fn, ta, tb, m, n, k, a, lda, b, ldb, c, dt):
    rc = fn(ta, tb, I64(m), I64(n), I64(k), I64(1), P(a.data_ptr), I64(lda), I64(0), P(b.data_ptr), I64(ldb),
            I64(0), P(c.data_ptr), I64(n), I64(0), DT[dt], DT[dt], F(1.0), None, 0, None)
    assert rc == 0, lib.sf_last_error()


# (dtype, transA, M, N, K, expected plan): NT split tail over 32 MB of the
# scratch, then a smaller TT split-K (8 MB), fp32 split-K (2 MB), and no
# split (fp32 small blocks, 16-bit tiles).
CASES = [
    ("bfloat16", 0, 4352, 4096, 4096, "gemm nt 256x256 lds-dma 16-bit persistent split-tail 16x8"),
    ("bfloat16", 1, 1024, 1024, 4096, "gemm tt 256x256 lds-dma 16-bit split-tail 16x8"),
    ("float32", 0, 64, 1000, 4096, "gemm tile 64x64 lds-dma fp32 split-tail 16x8"),
    ("float32", 0, 64, 512, 512, "gemm small 16x16 fp32"),
    ("float16", 0, 300, 200, 136, "gemm tile 64x64 16-bit"),
]


def _cu_count(lib):
    cus, mem, clk = ctypes.c_int(0), ctypes.c_int64(0), ctypes.c_int(0)
    dev = ctypes.c_int(0)
    assert lib.sf_get_device(ctypes.byref(dev)) == 0
    args = [ctypes.byref(cus), ctypes.byref(mem), ctypes.byref(clk)]
    assert lib.sf_get_device_props(dev, *args, None) == 0, lib.sf_last_error()
    return cus.value


def test_noalloc_matches_sf_gemm_in_sequence(lib):
    g = cu()
    if _cu_count(lib) != 256:
        pytest.skip("the expected plans are those of a 256-CU device")
    for dt, ta, m, n, k, want in CASES:
        print("noalloc case", dt, ta, m, n, k, flush=True)
        rng = np.random.default_rng(m + n + k)
        a = rnd(rng, (k, m) if ta else (m, k), 1.0, dt)
        b = rnd(rng, (n, k), 0.05, dt)
        ga, gb = up(a, dt), up(b, dt)
        c0 = up(np.zeros((m, n), np.float32), dt)
        c1 = up(np.full((m, n), np.nan, np.float32), dt)
        lda = m if ta else k
        assert _plan(lib, ta, 1, m, n, k, ga, lda, gb, k, c0, dt) == want
        _call(lib, lib.sf_gemm, ta, 1, m, n, k, ga, lda, gb, k, c0, dt)
        for rep in range(2):
            _call(lib, lib.sf_gemm_noalloc, ta, 1, m, n, k, ga, lda, gb, k, c1, dt)
            g.device_synchronize()
            y0 = g.gputensor_to_numpy(c0)
            y1 = g.gputensor_to_numpy(c1)
            assert np.array_equal(y0.view(np.uint32) if y0.dtype == np.float32 else y0.view(np.uint16),
                                  y1.view(np.uint32) if y1.dtype == np.float32 else y1.view(np.uint16)), (dt, m, n, k, rep)
        # and the values themselves, on a few rows, against fp64
        rows = np.r_[0, m // 2, m - 1]
        a_rows = (a.T if ta else a)[rows]
        y64 = ref.linear_f64(a_rows, b)
        yv = np.asarray(y1, np.float32)[rows]
        tol = 1e-5 * np.sqrt(k) * float(np.max(np.abs(y64))) if dt == "float32" else tol_16(k) * 8
        assert float(np.max(np.abs(yv - y64))) <= tol, (dt, m, n, k)


def test_noalloc_rejects_like_sf_gemm(lib):
    """Argument errors are the same as sf_gemm's, before any HIP call."""
    x = up(np.zeros((16, 16), np.float32), "bfloat16")
    rc = lib.sf_gemm_noalloc(0, 1, I64(-1), I64(16), I64(16), I64(1), P(x.data_ptr), I64(16), I64(0),
                             P(x.data_ptr), I64(16), I64(0), P(x.data_ptr), I64(16), I64(0), 2, 2, F(1.0), None, 0,
                             None)
    assert rc == -2 and b"negative size" in lib.sf_last_error()


def test_noalloc_allocates_nothing_in_a_fresh_process():
    """A child process that has run no split plan calls sf_gemm_noalloc on a
    split plan twice: the device's free bytes (hipMemGetInfo) and the
    library's split workspace are unchanged across those calls.  The same
    plan through sf_gemm then allocates its workspace, which both readings
    show, and its output is bit-identical to the no-allocation calls."""
    print("noalloc fresh process: 4352x4096x4096 bf16 persistent split", flush=True)
    r = subprocess.run([sys.executable, os.path.join(ROOT, "tests", "noalloc_fresh_process.py")],
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stdout + r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    print(out, flush=True)
    assert "split" in out["plan_split"] and "split" not in out["plan_warm"], out
    assert out["ws0"] == 0 and out["ws1"] == 0, out
    assert out["free1"] == out["free0"], out
    # sf_gemm's workspace: 16 tail tiles x 8 parts x 256 KB of partials + counters
    assert out["ws2"] >= 16 * 8 * 256 * 1024, out
    assert out["free0"] - out["free2"] >= out["ws2"], out
    assert out["bit_identical"], out


def test_noalloc_under_graph_capture(lib):
    """One uncaptured call on the device (it looks up the scratch address),
    then a split-plan sf_gemm_noalloc call captured on a stream into a HIP
    graph (its counters are cleared by a fill kernel, no memset node).  The
    graph replays three times, with eager work and a synchronisation
    between replays, and every replay is bit-identical to sf_gemm."""
    hip = ctypes.CDLL("libamdhip64.so")
    g = cu()
    m, n, k = 4352, 4096, 4096
    rng = np.random.default_rng(93)
    x = rnd(rng, (m, k), 1.0, "bfloat16")
    w = rnd(rng, (n, k), 1.0 / np.sqrt(k), "bfloat16")
    gx, gw = up(x, "bfloat16"), up(w, "bfloat16")
    c0 = up(np.zeros((m, n), np.float32), "bfloat16")
    c1 = up(np.full((m, n), np.nan, np.float32), "bfloat16")
    assert _plan(lib, 0, 1, m, n, k, gx, k, gw, k, c0, "bfloat16").endswith("split-tail 16x8")
    _call(lib, lib.sf_gemm, 0, 1, m, n, k, gx, k, gw, k, c0, "bfloat16")
    _call(lib, lib.sf_gemm_noalloc, 0, 1, m, n, k, gx, k, gw, k, c1, "bfloat16")
    g.device_synchronize()
    y0 = g.gputensor_to_numpy(c0).view(np.uint16)
    stream, graph, exe = P(), P(), P()
    assert lib.sf_stream_create(ctypes.byref(stream)) == 0
    try:
        print("noalloc graph capture: begin", flush=True)
        assert hip.hipStreamBeginCapture(stream, 0) == 0
        rc = lib.sf_gemm_noalloc(0, 1, I64(m), I64(n), I64(k), I64(1), P(gx.data_ptr), I64(k), I64(0),
                                 P(gw.data_ptr), I64(k), I64(0), P(c1.data_ptr), I64(n), I64(0), 2, 2, F(1.0),
                                 None, 0, stream)
        assert hip.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
        assert rc == 0, lib.sf_last_error()
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, ctypes.c_size_t(0)) == 0
        for rep in range(3):
            g.gputensor_from_numpy(np.full((m, n), np.nan, np.float32), -1, g.BFLOAT16)  # eager work
            fill = up(np.full((m, n), np.nan, np.float32), "bfloat16")
            assert lib.sf_memcpy_d2d(P(c1.data_ptr), P(fill.data_ptr), ctypes.c_size_t(m * n * 2), None) == 0
            g.device_synchronize()
            print("noalloc graph capture: replay", rep, flush=True)
            assert hip.hipGraphLaunch(exe, stream) == 0
            assert lib.sf_stream_synchronize(stream) == 0
            y1 = g.gputensor_to_numpy(c1).view(np.uint16)
            assert np.array_equal(y0, y1), rep
    finally:
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        if graph.value:
            hip.hipGraphDestroy(graph)
        lib.sf_stream_destroy(stream)
