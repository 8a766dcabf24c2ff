"""libsfgemm's host code under AddressSanitizer and UndefinedBehaviorSanitizer
(CPU only, no GPU): every csrc/*.hip is compiled as the library is (device
code for gfx950 at -O0: the check launches no kernel, and it builds five
times faster) with the sanitizers on the host side only, linked with
tests/asan/abi_host_check.cpp, which drives the C ABI's validation, the
kernel planner over more than ten thousand shapes, the no-allocation
entry point's scratch check and the runtime wrappers' failure paths.  Any
sanitizer report, or a failed expectation, fails the test."""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "scaffolding_amd", "csrc")
HOST_SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer"]


def _hipcc():
    for c in ("/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    return None


@pytest.mark.skipif(_hipcc() is None, reason="hipcc not available")
def test_host_code_under_asan_ubsan():
    hipcc = _hipcc()
    base = [hipcc, "--offload-arch=gfx950", "-O1", "-Xarch_device", "-O0", "-g", "-std=c++17",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-I", os.path.join(ROOT, "include"), "-I", CSRC, *HOST_SAN]
    with tempfile.TemporaryDirectory() as d:
        srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip"))) + [os.path.join(ROOT, "tests", "asan",
                                                                              "abi_host_check.cpp")]
        objs = [os.path.join(d, os.path.basename(s) + ".o") for s in srcs]

        def comp(so):
            s, o = so
            extra = ["-x", "hip"] if s.endswith(".hip") else []
            r = subprocess.run(base + extra + ["-c", s, "-o", o], capture_output=True, text=True, timeout=600)
            assert r.returncode == 0, r.stderr[-3000:]

        with cf.ThreadPoolExecutor(max_workers=8) as ex:
            list(ex.map(comp, zip(srcs, objs)))
        exe = os.path.join(d, "abi_host_check")
        r = subprocess.run([hipcc, "--offload-arch=gfx950", *HOST_SAN, "-o", exe, *objs], capture_output=True,
                           text=True, timeout=600)
        assert r.returncode == 0, r.stderr[-3000:]
        env = dict(os.environ, HIP_VISIBLE_DEVICES="-1", ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
                   UBSAN_OPTIONS="print_stacktrace=1")
        env.pop("SF_PLAN_CU_COUNT", None)
        r = subprocess.run([exe], capture_output=True, text=True, timeout=600, env=env)
        out = r.stdout + r.stderr
        assert r.returncode == 0, out[-4000:]
        assert "AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
        assert "all expectations hold" in r.stdout
