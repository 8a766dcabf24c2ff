"""The C ABI on the CPU (no GPU needed): libsfgemm loads, exports every
function include/sfgemm.h declares, validates arguments before touching the
device (the reference's error convention: 0 ok, negative code, text), and
the dispatcher picks the documented kernel for each config shape."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sfgemm.h")
LIB = os.path.join(ROOT, "scaffolding_amd", "libsfgemm.so")

I64 = ctypes.c_int64


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail("libsfgemm.so not built: run python scaffolding_amd/build.py")
    so = ctypes.CDLL(LIB)
    so.sf_last_error.restype = ctypes.c_char_p
    so.sf_status_string.restype = ctypes.c_char_p
    return so


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sf_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert len(names) >= 39
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_status_strings(lib):
    assert lib.sf_status_string(0) == b"success"
    assert lib.sf_status_string(-2) == b"invalid argument"
    assert lib.sf_status_string(-3) == b"unsupported operation"
    assert lib.sf_version() == 100


def gemm(lib, transA=0, transB=1, M=4, N=4, K=4, batch=1, A=256, lda=4, sA=0, B=512, ldb=4, sB=0,
         C=768, ldc=4, sC=0, ab=2, c=2, alpha=1.0, bias=None, epi=0):
    return lib.sf_gemm(transA, transB, I64(M), I64(N), I64(K), I64(batch), ctypes.c_void_p(A), I64(lda),
                       I64(sA), ctypes.c_void_p(B), I64(ldb), I64(sB), ctypes.c_void_p(C), I64(ldc),
                       I64(sC), ab, c, ctypes.c_float(alpha), ctypes.c_void_p(bias), epi, None)


@pytest.mark.parametrize("kw,code,text", [
    (dict(A=None), -2, b"null operand pointer"),
    (dict(C=None), -2, b"null operand pointer"),
    (dict(M=-1), -2, b"negative size"),
    (dict(transA=1, M=8, lda=4), -2, b"leading dimension"),
    (dict(ab=2, c=1), -3, b"output dtype"),
    (dict(ab=7), -2, b"unknown dtype"),
    (dict(epi=9), -2, b"unknown epilogue"),
    (dict(epi=1), -2, b"needs a bias"),
    (dict(bias=1024), -2, b"has no bias"),
    (dict(lda=3), -2, b"leading dimension"),
    (dict(transB=0, ldb=3), -2, b"leading dimension"),
    (dict(batch=2, sC=3), -2, b"overlaps batch"),
    (dict(M=1 << 31), -2, b"2^31"),
])
def test_gemm_validation_without_device(lib, kw, code, text):
    assert gemm(lib, **kw) == code
    assert text in lib.sf_last_error()


@pytest.mark.parametrize("args,ok", [
    ((0, -1, 0), True), ((3, 0, 16), True), ((7, 256, 2), True),
    ((8, -1, 0), False), ((-1, -1, 0), False), ((0, 257, 0), False), ((0, -1, 1), False),
    ((0, -1, 17), False),
])
def test_test_hooks_are_validated(lib, args, ok):
    """The test hooks are set only through sf_set_test_hooks (the library
    reads no environment variable for them) and are range-checked."""
    try:
        rc = lib.sf_set_test_hooks(*args)
        assert (rc == 0) == ok, (args, rc)
        if not ok:
            assert rc == -2 and b"sf_set_test_hooks" in lib.sf_last_error()
    finally:
        assert lib.sf_set_test_hooks(0, -1, 0) == 0


def test_library_reads_no_test_hook_from_the_environment():
    src = "".join(open(os.path.join(ROOT, "scaffolding_amd", "csrc", f)).read()
                  for f in os.listdir(os.path.join(ROOT, "scaffolding_amd", "csrc")))
    assert "SF_TEST_" not in src


def test_gemm_empty_is_noop(lib):
    assert gemm(lib, M=0, A=None, B=None, C=None) == 0
    assert gemm(lib, N=0, A=None, B=None, C=None) == 0
    assert gemm(lib, batch=0, A=None, B=None, C=None) == 0


def test_rowops_validation(lib):
    assert lib.sf_softmax_rows(None, None, I64(3), I64(4), 0, 0, ctypes.c_float(1.0), None) == -2
    assert lib.sf_softmax_rows(None, None, I64(0), I64(4), 0, 0, ctypes.c_float(1.0), None) == 0
    assert lib.sf_silu(None, None, I64(-1), 0, None) == -2
    assert lib.sf_cast(None, 0, None, 5, I64(1), None) == -2
    assert lib.sf_bias_add_rows(None, None, I64(2), I64(2), 0, None) == -2
    assert lib.sf_sum_dim(None, None, I64(1), I64(4), I64(3), 0, 0, None) == -2
    assert b"null pointer" in lib.sf_last_error()
    assert lib.sf_sum_dim(None, None, I64(0), I64(4), I64(3), 0, 0, None) == 0
    assert lib.sf_sum_dim(None, None, I64(1), I64(-1), I64(3), 0, 0, None) == -2
    assert lib.sf_sum_dim(None, None, I64(1), I64(4), I64(3), 2, 1, None) == -3
    U64 = ctypes.c_uint64
    drop = lambda n, p, dt=0: lib.sf_dropout(None, None, None, I64(n), dt, ctypes.c_float(p), U64(0), U64(0), None)
    assert drop(4, 0.5) == -2                    # null pointers
    assert drop(4, 1.0) == -2 and b"p must be" in lib.sf_last_error()
    assert drop(4, -0.1) == -2
    assert drop(4, float("nan")) == -2
    assert drop(-1, 0.5) == -2
    assert drop(4, 0.5, dt=7) == -2              # unknown dtype
    assert drop(0, 0.5) == 0                     # empty: nothing to do


def plan(**kw):
    from scaffolding_amd import _cuda_ops as cu
    a = dict(transB=1, M=4096, N=4096, K=4096, batch=1, ptr_a=256, lda=4096, stride_a=0, ptr_b=512,
             ldb=4096, stride_b=0, ldc=4096, stride_c=0, dtype="bfloat16")
    a.update(kw)
    return cu.gemm_plan(a["transB"], a["M"], a["N"], a["K"], a["batch"], a["ptr_a"], a["lda"], a["stride_a"],
                        a["ptr_b"], a["ldb"], a["stride_b"], a["ldc"], a["stride_c"], a["dtype"],
                        transA=a.get("transA", 0))


def test_dispatch_for_config_shapes():
    # north star / C3 M=4096 / C5: large NT -> 8-wave ping-pong kernel
    assert plan().startswith("gemm nt 256x256 lds-dma")
    assert plan(M=4096, N=11008, ldc=11008).startswith("gemm nt 256x256 lds-dma")
    assert plan(M=17776, N=1920, K=7680, lda=7680, ldb=7680, ldc=1920).startswith("gemm nt 256x256 lds-dma")
    # C5 tails (560 / 1610 / 2100 tiles): persistent tiles (more tiles than
    # CUs, last round at most half full); behind whole waves K >= 4096
    # splits the last wave (MLP-down), and so does K >= 1280 in a launch of
    # under 3 rounds, in parts of at least 5 k-units (out-projection: 15
    # units, 3 parts); QKV and MLP-up (6-8 rounds) run it unsplit
    assert plan(M=17776, N=1920, K=7680, lda=7680, ldb=7680, ldc=1920) \
        == "gemm nt 256x256 lds-dma 16-bit persistent split-tail 48x5"
    assert plan(M=17776, N=1920, K=1920, lda=1920, ldb=1920, ldc=1920) \
        == "gemm nt 256x256 lds-dma 16-bit persistent split-tail 48x3"
    # below 10 k-units a short launch stays unsplit
    assert plan(M=17776, N=1920, K=1024, lda=1024, ldb=1024, ldc=1920) \
        == "gemm nt 256x256 lds-dma 16-bit persistent"
    assert plan(M=4352, N=7936, K=1024, lda=1024, ldb=1024, ldc=7936) \
        == "gemm nt 256x256 lds-dma 16-bit persistent"
    assert plan(M=17776, N=1920, K=1280, lda=1280, ldb=1280, ldc=1920) \
        == "gemm nt 256x256 lds-dma 16-bit persistent split-tail 48x2"
    assert plan(M=17776, N=5760, K=1920, lda=1920, ldb=1920, ldc=5760) \
        == "gemm nt 256x256 lds-dma 16-bit persistent"
    assert plan(M=17776, N=7680, K=1920, lda=1920, ldb=1920, ldc=7680) \
        == "gemm nt 256x256 lds-dma 16-bit persistent"
    # one tile per CU (north star) and a last round more than half full
    # (C3 M = 4096: 688 tiles) keep one workgroup per tile, on the
    # one-wave-per-SIMD kernel (K >= 4096, C rows of whole 128-byte lines)
    assert plan() == "gemm nt 256x256 lds-dma 16-bit 4-wave"
    assert plan(M=4096, N=11008, ldc=11008) == "gemm nt 256x256 lds-dma 16-bit 4-wave"
    assert plan(K=2048, lda=2048, ldb=2048) == "gemm nt 256x256 lds-dma 16-bit"
    assert plan(N=4000, ldc=4000) == "gemm nt 256x256 lds-dma 16-bit"
    assert plan(N=4000, ldc=4032) == "gemm nt 256x256 lds-dma 16-bit 4-wave"
    # whole rounds only: persistent; a split tail packs each XCD with at most
    # 32 parts (85 tail tiles: 11 on the busiest XCD, so 2 parts each)
    assert plan(N=8192, K=512, lda=512, ldb=512, ldc=8192) == "gemm nt 256x256 lds-dma 16-bit persistent"
    assert plan(M=7900, N=2800, K=4352, lda=4352, ldb=4352, ldc=2800) \
        == "gemm nt 256x256 lds-dma 16-bit persistent split-tail 85x2"
    # backward layouts keep one workgroup per tile or split part
    assert plan(transA=1, transB=0, M=4352, N=4096, K=4096, lda=4352, ldb=4096) \
        == "gemm tn 256x256 lds-dma 16-bit split-tail 16x8"
    # C3 decode shapes -> row-segment stream kernel (K = 512 x waves)
    assert plan(M=1, N=11008, ldc=11008).startswith("gemm skinny line")
    assert plan(M=16, N=11008, ldc=11008).startswith("gemm skinny line")
    # other K: the chunked stream kernel
    assert plan(M=16, N=1920, K=1920, lda=1920, ldb=1920, ldc=1920) == "gemm skinny 16-bit"
    # C4: QK^T (K = 64: the store-bound 128 x 128 kernel) and P.V (N = 64, B N-contiguous)
    assert plan(M=4096, N=4096, K=64, batch=60, lda=64, ldb=64, stride_a=4096 * 64, stride_b=4096 * 64,
                stride_c=4096 * 4096, dtype="float16") == "gemm nt 128x128 k64 lds-dma 16-bit"
    assert plan(transB=0, M=4096, N=64, K=4096, batch=60, ldb=64, ldc=64, stride_a=4096 * 4096,
                stride_b=4096 * 64, stride_c=4096 * 64, dtype="float16").startswith("gemm tile 256x64")
    # C1 / C2 fp32: outputs of at most CUs / 4 tiles of 64 x 64 with
    # K <= 2048 -> small-block kernel (16 x 16 blocks up to half the CUs,
    # then 16 x 32); K-contiguous A, K % 32 == 0 -> LDS-DMA 64 x 64 with two
    # k-groups (one k-group, split-K, for few tiles and K > 2048); otherwise
    # the register-staged tiles
    assert plan(M=64, N=512, K=512, lda=512, ldb=512, ldc=512, dtype="float32") == "gemm small 16x16 fp32"
    assert plan(transB=0, M=512, N=512, K=512, lda=512, ldb=512, ldc=512, dtype="float32") \
        == "gemm small 16x32 fp32"
    assert plan(transB=0, M=1024, N=1024, K=1024, lda=1024, ldb=1024, ldc=1024, dtype="float32") \
        == "gemm tile 64x64 lds-dma k-groups fp32"
    assert plan(transB=0, dtype="float32") == "gemm tile 64x64 lds-dma k-groups fp32"
    assert plan(M=64, dtype="float32") == "gemm tile 64x64 lds-dma fp32 split-tail 64x4"
    assert plan(M=4096, K=4064, lda=4064, ldb=4064, dtype="float32") == "gemm tile 64x64 lds-dma fp32"
    assert plan(K=4004, lda=4004, ldb=4004, dtype="float32").startswith("gemm tile 128x128 fp32")
    assert plan(transB=0, M=768, N=768, K=1024, lda=1024, ldb=768, ldc=768, dtype="float32") \
        == "gemm tile 64x64 lds-dma k-groups fp32"
    assert plan(transB=0, M=200, N=300, K=4096, lda=4096, ldb=300, ldc=300, dtype="float32") \
        == "gemm tile 64x64 lds-dma fp32 split-tail 20x8"
    assert plan(M=1000, N=900, K=100, lda=100, ldb=100, ldc=900, dtype="float32") == "gemm tile 64x64 fp32"
    assert plan(M=300, N=260, K=1000, lda=1000, ldb=1000, ldc=260, dtype="float32") == "gemm small 16x32 fp32"
    # backward GEMMs: dW = dY^T X (A stored K x M) takes the register-staged
    # tiles, never the LDS-DMA or skinny kernels; dX = dY W is NN
    assert plan(transA=1, transB=0, M=1920, N=7680, K=17776, lda=1920, ldb=7680, ldc=7680) \
        == "gemm tn 256x256 lds-dma 16-bit"
    assert plan(transA=1, transB=0, M=1920, N=1920, K=17776, lda=1920, ldb=1920, ldc=1920) \
        == "gemm tn 256x256 lds-dma 16-bit split-tail 64x4"
    assert plan(transA=1, transB=0, ldb=4096) == "gemm tn 256x256 lds-dma 16-bit"
    assert plan(transA=0, transB=0, ldb=4096) == "gemm nn 256x256 lds-dma 16-bit"
    # dX (NN) with more tiles than CUs: persistent tiles, split tails as NT
    # (C5 QKV / out-projection / MLP-down dX shapes)
    assert plan(transA=0, transB=0, M=17776, N=1920, K=5760, lda=5760, ldb=1920, ldc=1920) \
        == "gemm nn 256x256 lds-dma 16-bit persistent split-tail 48x5"
    assert plan(transA=0, transB=0, M=17776, N=1920, K=1920, lda=1920, ldb=1920, ldc=1920) \
        == "gemm nn 256x256 lds-dma 16-bit persistent split-tail 48x3"
    assert plan(transA=0, transB=0, M=17776, N=7680, K=1920, lda=1920, ldb=7680, ldc=7680) \
        == "gemm nn 256x256 lds-dma 16-bit persistent"
    # dW (TN) stays one workgroup per tile
    assert plan(transA=1, transB=0, M=5760, N=1920, K=17776, lda=5760, ldb=1920, ldc=1920) \
        == "gemm tn 256x256 lds-dma 16-bit"
    assert plan(transA=1, transB=1) == "gemm tt 256x256 lds-dma 16-bit"
    assert plan(transA=1, transB=0, ldb=4096, K=4000) == "gemm tn 256x256 lds-dma 16-bit"  # any K for TN
    assert plan(transA=0, transB=0, ldb=4096, K=4000) == "gemm tile 256x256 16-bit"  # K % 128 != 0
    assert plan(transA=1, transB=1, M=16, N=11008, ldc=11008, lda=16) == "gemm tile 64x64 16-bit"
    assert plan(transA=1, transB=0, M=4092, lda=4092).startswith("gemm tile generic")
    assert plan(transA=1, transB=0, dtype="float32").startswith("gemm tile 128x128 fp32")
    # unaligned operands fall back to the bounds-checked kernel
    assert plan(K=4095, lda=4095, ldb=4095).startswith("gemm tile generic")
    assert plan(ptr_a=258).startswith("gemm tile generic")


def test_python_surface_without_device():
    import numpy as np

    import scaffolding_amd as sf
    assert sf.dtype.from_any("bfloat16") is sf.bfloat16
    assert sf.dtype.from_any(np.float16) is sf.float16
    assert sf.bfloat16.to_numpy() == np.float32  # host view, as reference dtype.py:31
    assert str(sf.device("cuda:1")) == "cuda:1" and sf.device("cuda") == sf.device("cuda:0")
    t = sf.tensor(np.ones((2, 3), np.float32))
    assert t.shape == (2, 3) and t.dtype is sf.float32 and not t.is_cuda
    with pytest.raises(RuntimeError, match="GPU only"):
        sf.matmul(t, t)
    with pytest.raises(RuntimeError, match="GPU only"):
        sf.nn.functional.linear(t, t)
    with pytest.raises(TypeError):
        sf.tensor(np.ones(3), dtype="bfloat16")
    assert sf.cuda.device_count() >= 0


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_split_tail_needs_whole_tiles_per_xcd():
    """The tail split hands every XCD (tiles - tail) / 8 whole tiles, so it
    is planned only when that divides evenly; the persistent kernel needs a
    CU count that is a multiple of 8.  Run in a fresh process with the
    host-only CU-count override (no device visible): M = 17776, N = 1920,
    K = 7680 is 560 tiles; on 248 CUs 496 whole tiles remain (persistent,
    split: at most 31 parts per XCD, 8 tail tiles on each, so 3 parts), on
    250 CUs 500 (neither persistent nor split: one workgroup per tile, on
    the one-wave-per-SIMD kernel)."""
    code = ("import ctypes,sys;so=ctypes.CDLL(sys.argv[1]);b=ctypes.create_string_buffer(96);I=ctypes.c_int64;"
            "rc=so.sf_gemm_plan(0,1,I(17776),I(1920),I(7680),I(1),ctypes.c_void_p(256),I(7680),I(0),"
            "ctypes.c_void_p(512),I(7680),I(0),ctypes.c_void_p(1024),I(1920),I(0),2,2,ctypes.c_float(1.0),"
            "None,0,b,96);print(rc, b.value.decode())")
    got = {}
    for cus in (248, 250, 256):
        env = dict(os.environ, SF_PLAN_CU_COUNT=str(cus), HIP_VISIBLE_DEVICES="-1")
        r = subprocess.run([sys.executable, "-c", code, LIB], capture_output=True, text=True, timeout=120, env=env)
        assert r.returncode == 0, r.stderr
        got[cus] = r.stdout.strip()
    assert got[256] == "0 gemm nt 256x256 lds-dma 16-bit persistent split-tail 48x5"
    assert got[248] == "0 gemm nt 256x256 lds-dma 16-bit persistent split-tail 64x3"
    assert got[250] == "0 gemm nt 256x256 lds-dma 16-bit 4-wave"


def test_noalloc_rejects_plans_beyond_its_scratch():
    """sf_gemm_noalloc runs sf_gemm's plans from a fixed scratch array; a plan
    whose workspace would not fit is refused with a clear error before any
    HIP call.  No 256-CU plan is that large, so a fresh process plans for
    1024 CUs (host-only override): TN 2816 x 2816 x 4096 then splits 121
    tiles 8 ways, 242 MB of partials."""
    code = ("import ctypes,sys;so=ctypes.CDLL(sys.argv[1]);so.sf_last_error.restype=ctypes.c_char_p;"
            "I=ctypes.c_int64;P=ctypes.c_void_p;"
            "rc=so.sf_gemm_noalloc(1,0,I(2816),I(2816),I(4096),I(1),P(256),I(2816),I(0),P(512),I(2816),I(0),"
            "P(1024),I(2816),I(0),2,2,ctypes.c_float(1.0),None,0,None);print(rc, so.sf_last_error().decode())")
    env = dict(os.environ, SF_PLAN_CU_COUNT="1024", HIP_VISIBLE_DEVICES="-1")
    r = subprocess.run([sys.executable, "-c", code, LIB], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0, r.stderr
    rc, msg = r.stdout.strip().split(" ", 1)
    assert int(rc) == -3 and "scratch" in msg and "253755392" in msg, r.stdout
