"""In-tree build of the package's native parts.

1. every ``csrc/*.hip`` -> object with ``hipcc --offload-arch=gfx950``
   (parallel), linked into ``scaffolding_amd/libsfgemm.so``;
2. ``_cuda_ops.pyx`` -> C with Cython -> ``_cuda_ops*.so`` with the host C
   compiler, linked against libsfgemm.so through an ``$ORIGIN`` rpath;
3. ``probes/*.hip`` -> ``scaffolding_amd/libsfprobe.so``: hardware
   measurement kernels that ``bench.py --hw-probes`` runs.  No product path
   loads it.

Run ``python scaffolding_amd/build.py`` (or ``__graft_entry__.build()``).
Artefacts stay in the source tree (git-ignored) so they travel with it.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys
import sysconfig

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libsfgemm.so")

ARCH = os.environ.get("SF_OFFLOAD_ARCH", "gfx950")
# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in generated code.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build libsfgemm")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError("build step failed (%d): %s\n%s" % (proc.returncode, " ".join(cmd), proc.stdout))


def build_lib(jobs: int | None = None, verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    hipcc = _hipcc()
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    objs = []
    cmds = []
    for src in sources:
        obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, "-I", INCLUDE, "-c", src, "-o", obj])
    jobs = jobs or min(len(cmds), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        for cmd, fut in zip(cmds, [ex.submit(_run, c) for c in cmds]):
            fut.result()
            if verbose:
                print("compiled", cmd[-3], flush=True)
    tmp = LIB + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    return LIB


def build_ext(verbose: bool = False) -> str:
    import numpy as np
    from Cython.Build import cythonize  # noqa: F401  (ensures Cython is importable)

    os.makedirs(BUILD, exist_ok=True)
    pyx = os.path.join(PKG, "_cuda_ops.pyx")
    c_out = os.path.join(BUILD, "_cuda_ops.c")
    _run([sys.executable, "-m", "cython", "-3", "-I", INCLUDE, pyx, "-o", c_out])
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    target = os.path.join(PKG, "_cuda_ops" + suffix)
    cc = os.environ.get("CC", "gcc")
    tmp = target + ".tmp"
    _run([
        cc, "-O2", "-fPIC", "-shared", "-Wno-unused-function",
        "-DNPY_NO_DEPRECATED_API=NPY_1_7_API_VERSION",
        "-I", sysconfig.get_paths()["include"], "-I", np.get_include(), "-I", INCLUDE,
        c_out, "-o", tmp, "-L", PKG, "-lsfgemm", "-Wl,-rpath,$ORIGIN",
    ])
    os.replace(tmp, target)
    if verbose:
        print("built", target, flush=True)
    return target


def build_probes(verbose: bool = False) -> str:
    sources = sorted(glob.glob(os.path.join(PKG, "probes", "*.hip")))
    target = os.path.join(PKG, "libsfprobe.so")
    tmp = target + ".tmp"
    _run([_hipcc(), *HIPCC_FLAGS, "-shared", "-o", tmp, *sources])
    os.replace(tmp, target)
    if verbose:
        print("built", target, flush=True)
    return target


def build(verbose: bool = False) -> None:
    build_lib(verbose=verbose)
    build_ext(verbose=verbose)
    build_probes(verbose=verbose)


if __name__ == "__main__":
    build(verbose=True)
