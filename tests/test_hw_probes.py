"""The hardware measurement kernels (scaffolding_amd/probes/hw_probes.hip,
libsfprobe.so) that bench.py --hw-probes runs: each result must sit where
the hardware's documented rates put it, so the probes measure what their
tables say.  Not part of the GEMM library's product path."""
import ctypes
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "scaffolding_amd", "libsfprobe.so")


def _lib():
    if not os.path.exists(LIB):
        pytest.fail("libsfprobe.so is not built (run __graft_entry__.build())")
    return ctypes.CDLL(LIB)


def test_probe_library_exports():
    lib = _lib()
    for name in ("sfp_issue", "sfp_mfma_rate", "sfp_lds_read"):
        assert hasattr(lib, name), name


def test_probe_rejects_bad_arguments_without_a_gpu_call():
    lib = _lib()
    cyc = (ctypes.c_double * 2)()
    assert lib.sfp_issue(9, -1, 10, cyc) == 1      # no such stream
    assert lib.sfp_issue(1, 0, 10, cyc) == 1       # 0 is not a second stream
    assert lib.sfp_issue(1, 4, 10, cyc) == 1       # a pair the library does not hold
    assert lib.sfp_issue(1, -1, 0, cyc) == 1
    us, fl = ctypes.c_double(), ctypes.c_double()
    assert lib.sfp_mfma_rate(1, 0, 0, ctypes.byref(us), ctypes.byref(fl)) == 1
    bpn = ctypes.c_double()
    assert lib.sfp_lds_read(0, 1, ctypes.byref(bpn)) == 1


def _issue(lib, a, b, iters=500):
    cyc = (ctypes.c_double * 2)()
    rc = lib.sfp_issue(a, b, iters, cyc)
    assert rc == 0, rc
    return cyc[0], cyc[1]


@pytest.mark.gpu
def test_issue_streams_sit_at_their_pipe_bounds():
    lib = _lib()
    # 16 MFMAs of 16 cycles each: the matrix pipe's bound, and not far above
    mfma, _ = _issue(lib, 1, -1)
    assert 16 * 16 * 0.97 <= mfma <= 16 * 16 * 1.5, mfma
    # two MFMA waves share one pipe: the later one needs both waves' MFMAs
    a, b = _issue(lib, 1, 1)
    assert max(a, b) >= 2 * 16 * 16 * 0.97, (a, b)
    # v_exp_f32 at half rate at best: 32 of them take at least 32 x 8 cycles
    e, _ = _issue(lib, 3, -1)
    assert e >= 32 * 8 * 0.97, e
    # 64 FMAs of one wave: at least 64 x 2 cycles (32 lanes a cycle)
    f, _ = _issue(lib, 2, -1)
    assert f >= 64 * 2 * 0.97, f


@pytest.mark.gpu
def test_mfma_rate_is_at_most_peak_and_constant_operands_run_faster():
    lib = _lib()
    out = {}
    for random in (1, 0):
        us, fl = ctypes.c_double(), ctypes.c_double()
        assert lib.sfp_mfma_rate(random, 200, 50, ctypes.byref(us), ctypes.byref(fl)) == 0
        assert fl.value == 2.0 * 4096 ** 3
        out[random] = fl.value / (us.value * 1e-6)
    # the datasheet's dense bf16 peak (2.5 PF at 2.4 GHz); the part may boost a little past it
    assert out[0] <= 2.5e15 * 1.06, out
    assert out[1] <= out[0] * 1.02, out


@pytest.mark.gpu
def test_lds_read_rate_is_positive_and_below_256_bytes_per_clock():
    lib = _lib()
    bpn = ctypes.c_double()
    assert lib.sfp_lds_read(2000, 3, ctypes.byref(bpn)) == 0
    # at most 256 B per clock per CU at 2.4 GHz
    assert 0 < bpn.value <= 256 * 2.4 * 1.06, bpn.value
