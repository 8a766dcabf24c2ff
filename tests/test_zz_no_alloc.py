"""sf_gemm_noalloc (the entry point that allocates nothing: its split plans
take their workspace from a fixed per-device scratch array) against
sf_gemm on the same inputs: the same plans, so the outputs must be
bit-identical.  Two split calls in a row, the second on a smaller problem,
then fp32 split-K and an unsplit shape; each noalloc call runs twice, so
the counters the first call leaves behind are shown to be cleared."""
from __future__ import annotations

import ctypes
import os

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


def test_noalloc_matches_sf_gemm_in_sequence(lib):
    g = cu()
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
