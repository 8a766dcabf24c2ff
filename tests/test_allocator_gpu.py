"""Native caching allocator (reference _cuda_ops.pyx:413-437 keeps a pool of
freed device blocks keyed by size): reuse of freed blocks, the pooled-bytes
limit, and eviction of the least recently used sizes when a new workload's
sizes would push the pool over the limit."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import cu

pytestmark = pytest.mark.gpu

MIB = 1 << 20
DEFAULT_LIMIT = 16 << 30


@pytest.fixture
def small_pool():
    g = cu()
    g.device_synchronize()
    g.empty_cache()
    g.set_cache_limit(64 * MIB)
    try:
        yield g
    finally:
        g.set_cache_limit(DEFAULT_LIMIT)
        g.empty_cache()


def _buf(g, mib):
    return g.empty((mib * MIB // 4,), np.float32)


def test_freed_block_is_reused(small_pool):
    g = small_pool
    a = _buf(g, 8)
    p = a.data_ptr
    del a
    assert g.cache_stats()[0] == 8 * MIB
    b = _buf(g, 8)
    assert b.data_ptr == p
    assert g.cache_stats()[0] == 0
    del b


def test_new_sizes_evict_least_recently_used(small_pool):
    g = small_pool
    old = [_buf(g, 16) for _ in range(3)]
    del old
    assert g.cache_stats()[0] == 48 * MIB
    new = [_buf(g, 24) for _ in range(2)]
    # 48 + 24 > 64: one 16 MiB block is evicted, then one more for the
    # second 24 MiB block, so both new blocks stay pooled.
    del new
    assert g.cache_stats()[0] == 64 * MIB
    again = [_buf(g, 24) for _ in range(2)]
    assert g.cache_stats()[0] == 16 * MIB
    del again
    assert g.cache_stats()[0] == 64 * MIB


def test_block_over_limit_is_not_pooled(small_pool):
    g = small_pool
    a = _buf(g, 4)
    del a
    big = _buf(g, 96)
    del big
    assert g.cache_stats()[0] == 4 * MIB


def test_contents_survive_eviction(small_pool):
    g = small_pool
    keep = g.gputensor_from_numpy(np.arange(1 << 20, dtype=np.float32))
    tmp = [_buf(g, 20) for _ in range(3)]
    del tmp
    tmp = [_buf(g, 30) for _ in range(2)]
    del tmp
    np.testing.assert_array_equal(g.gputensor_to_numpy(keep), np.arange(1 << 20, dtype=np.float32))


def test_allocation_failure_raises_and_leaves_the_library_usable():
    """An allocation the device cannot satisfy (64 TiB) fails the reference's
    way: the C ABI returns a negative code (SF_ERR_OOM) with the detail in
    sf_last_error, and the seam raises RuntimeError("CUDA error: ...")
    (reference _cuda_kernels.cuh:303-319, _cuda_ops.pyx:292-300).  The
    failure is not sticky: the next allocation and GEMM succeed."""
    import ctypes
    import os

    g = cu()
    with pytest.raises(RuntimeError, match="CUDA error: .*hipMalloc"):
        g.empty((1 << 44,), np.float32)
    lib = ctypes.CDLL(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                   "scaffolding_amd", "libsfgemm.so"))
    lib.sf_last_error.restype = ctypes.c_char_p
    p = ctypes.c_void_p()
    got = ctypes.c_size_t()
    rc = lib.sf_cache_alloc(0, ctypes.c_size_t(1 << 46), ctypes.byref(p), ctypes.byref(got))
    assert rc == -5 and p.value is None and b"out of memory" in lib.sf_last_error().lower()
    a = g.gputensor_from_numpy(np.eye(64, dtype=np.float32), 0, np.float32)
    y = g.gputensor_to_numpy(g.dev_matmul(a, a))
    assert np.array_equal(y, np.eye(64, dtype=np.float32))
