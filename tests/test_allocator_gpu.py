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
