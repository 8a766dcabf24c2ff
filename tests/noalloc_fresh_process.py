"""Run by tests/test_zz_no_alloc.py in a fresh child process, so no split
plan has run on the device before: shows that sf_gemm_noalloc allocates no
device memory, then that sf_gemm's split workspace does show up in the same
measurement.  Prints one JSON line.

Order: upload the operands (the caching allocator allocates them), one
uncaptured sf_gemm_noalloc call without a split (loads the code object and
looks up the scratch address), synchronise, read the device's free bytes
and the library's split workspace; two split-plan sf_gemm_noalloc calls,
synchronise, read both again; one sf_gemm call of the same plan (it
allocates the workspace), synchronise, read again.  Outputs are copied
back only after the last reading."""
from __future__ import annotations

import ctypes
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for p in (ROOT, HERE):
    if p not in sys.path:
        sys.path.insert(0, p)

from helpers import cu, rnd, up  # noqa: E402

I64, P, F, SZ = ctypes.c_int64, ctypes.c_void_p, ctypes.c_float, ctypes.c_size_t


def main() -> None:
    g = cu()
    lib = ctypes.CDLL(os.path.join(ROOT, "scaffolding_amd", "libsfgemm.so"))
    lib.sf_last_error.restype = ctypes.c_char_p
    g.set_device(0)

    def gemm(fn, m, n, k, a, b, c):
        rc = fn(0, 1, I64(m), I64(n), I64(k), I64(1), P(a.data_ptr), I64(k), I64(0), P(b.data_ptr), I64(k),
                I64(0), P(c.data_ptr), I64(n), I64(0), 2, 2, F(1.0), None, 0, None)
        if rc != 0:
            raise RuntimeError(lib.sf_last_error().decode())

    def plan(m, n, k, a, b, c):
        buf = ctypes.create_string_buffer(96)
        rc = lib.sf_gemm_plan(0, 1, I64(m), I64(n), I64(k), I64(1), P(a.data_ptr), I64(k), I64(0), P(b.data_ptr),
                              I64(k), I64(0), P(c.data_ptr), I64(n), I64(0), 2, 2, F(1.0), None, 0, buf, 96)
        if rc != 0:
            raise RuntimeError(lib.sf_last_error().decode())
        return buf.value.decode()

    def reading():
        free, total, ws = SZ(0), SZ(0), SZ(0)
        if lib.sf_device_synchronize() != 0 or lib.sf_mem_get_info(ctypes.byref(free), ctypes.byref(total)) != 0 \
                or lib.sf_workspace_bytes(0, ctypes.byref(ws)) != 0:
            raise RuntimeError(lib.sf_last_error().decode())
        return int(free.value), int(ws.value)

    m, n, k = 4352, 4096, 4096
    rng = np.random.default_rng(91)
    x = rnd(rng, (m, k), 1.0, "bfloat16")
    w = rnd(rng, (n, k), 1.0 / np.sqrt(k), "bfloat16")
    gx, gw = up(x, "bfloat16"), up(w, "bfloat16")
    c_noalloc = up(np.full((m, n), np.nan, np.float32), "bfloat16")
    c_gemm = up(np.zeros((m, n), np.float32), "bfloat16")
    warm = up(np.zeros((256, 256), np.float32), "bfloat16")
    out = {"plan_split": plan(m, n, k, gx, gw, c_gemm), "plan_warm": plan(256, 256, 256, gx, gw, warm)}

    gemm(lib.sf_gemm_noalloc, 256, 256, 256, gx, gw, warm)
    out["free0"], out["ws0"] = reading()
    gemm(lib.sf_gemm_noalloc, m, n, k, gx, gw, c_noalloc)
    gemm(lib.sf_gemm_noalloc, m, n, k, gx, gw, c_noalloc)
    out["free1"], out["ws1"] = reading()
    gemm(lib.sf_gemm, m, n, k, gx, gw, c_gemm)
    out["free2"], out["ws2"] = reading()

    y0 = g.gputensor_to_numpy(c_gemm).view(np.uint16)
    y1 = g.gputensor_to_numpy(c_noalloc).view(np.uint16)
    out["bit_identical"] = bool(np.array_equal(y0, y1))
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
