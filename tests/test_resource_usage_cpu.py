"""Register budget of the hot kernels, checked at compile time (CPU only).

The hot kernels are sized to fit their register budgets exactly (two waves
per SIMD: <= 256 VGPRs); a change that pushes one of them past it makes the
compiler spill to scratch memory, which costs a global-memory round trip per
spilled access.  This test compiles the hot translation units for gfx950
with the compiler's resource-usage report and fails on any scratch use by
the ping-pong GEMM (gemm16nt_pp), the row-segment skinny stream (skinny16l),
the fused attention (attn64) and the fp32 LDS-DMA and small-block GEMMs
(gemm32dma, gemm32small)."""
from __future__ import annotations

import concurrent.futures as cf
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "scaffolding_amd", "csrc")
HOT = ["gemm16_bf16.hip", "gemm16_f16.hip", "attention.hip", "gemm32.hip"]
WATCH = re.compile(r"gemm16nt_pp_kernel|gemm16nt_4w_kernel|gemm16nt_k64_kernel|skinny16l_kernel|attn64_kernel|gemm32dma_kernel|gemm32small_kernel")


def _hipcc():
    for c in ("/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    return None


def _report(src: str, out_dir: str) -> str:
    cmd = [_hipcc(), "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-I", os.path.join(ROOT, "include"), "--offload-device-only", "-c",
           os.path.join(CSRC, src), "-o", os.path.join(out_dir, src + ".o"),
           "-Rpass-analysis=kernel-resource-usage"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    return r.stderr


def _kernels(report: str):
    """(kernel name, VGPRs, scratch bytes per lane) from the remarks."""
    out, name, vgpr = [], None, None
    for line in report.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name, vgpr = m.group(1), None
            continue
        m = re.search(r"\bVGPRs: (\d+)", line)
        if m and name:
            vgpr = int(m.group(1))
            continue
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and name:
            out.append((name, vgpr, int(m.group(1))))
            name = None
    return out


@pytest.mark.skipif(_hipcc() is None, reason="hipcc not available")
def test_hot_kernels_do_not_spill():
    with tempfile.TemporaryDirectory() as d:
        with cf.ThreadPoolExecutor(max_workers=len(HOT)) as ex:
            reports = list(ex.map(lambda s: _report(s, d), HOT))
    seen = [k for r in reports for k in _kernels(r) if WATCH.search(k[0])]
    names = " ".join(k[0] for k in seen)
    for want in ("gemm16nt_pp_kernel", "gemm16nt_4w_kernel", "gemm16nt_k64_kernel", "skinny16l_kernel", "attn64_kernel", "gemm32dma_kernel",
                 "gemm32small_kernel"):
        assert want in names, "no %s instantiation found in the report" % want
    spilled = [k for k in seen if k[2] > 0]
    assert not spilled, "kernels using scratch (name, VGPRs, bytes/lane): %s" % spilled
    assert all(k[1] is not None and k[1] <= 256 for k in seen if "pp_kernel" in k[0] or "attn64" in k[0])
    # four workgroups of four waves per CU
    assert all(k[1] is not None and k[1] <= 128 for k in seen if "k64_kernel" in k[0])
