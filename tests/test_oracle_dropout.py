"""The dropout oracle (oracle/dropout.py) on the CPU: its Philox4x32-10
against the published Random123 known-answer vectors (Salmon, Moraes,
Dror, Shaw, SC 2011; kat_vectors of the Random123 distribution), and the
keep rule's law (each element kept with probability 1 - p, kept values
scaled by 1 / (1 - p)) against the binomial distribution."""
import numpy as np
import pytest

from oracle import dropout as D

# counter (4 words), key (2 words) -> output (4 words)
KAT = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff, 0xffffffff, 0xffffffff, 0xffffffff), (0xffffffff, 0xffffffff),
     (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
]


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_philox_known_answers(ctr, key, want):
    got = D.philox4x32_10(np.array(ctr, np.uint32), np.array(key, np.uint32))
    assert [int(v) for v in got] == list(want)


def test_philox_batched_equals_single():
    rng = np.random.default_rng(0)
    ctr = rng.integers(0, 2**32, (50, 4), dtype=np.uint64).astype(np.uint32)
    key = np.array([0x12345678, 0x9abcdef0], np.uint32)
    batch = D.philox4x32_10(ctr, key)
    for i in range(0, 50, 7):
        assert np.array_equal(batch[i], D.philox4x32_10(ctr[i], key))


def test_uniform_stream_layout():
    # element i uses word i % 4 of the block for counter (i // 4, 0, offset)
    seed, off = 0x1234_5678_9abc_def0, 0x0000_0002_0000_0003
    u = D.uniforms(9, seed, off)
    key = np.array([seed & 0xffffffff, seed >> 32], np.uint32)
    for g in range(3):
        r = D.philox4x32_10(np.array([g, 0, off & 0xffffffff, off >> 32], np.uint32), key)
        for q in range(4):
            if 4 * g + q < 9:
                assert u[4 * g + q] == (int(r[q]) >> 8) * 2.0 ** -24
    assert np.all((u >= 0) & (u < 1))


@pytest.mark.parametrize("p", [0.1, 0.5, 0.9])
def test_keep_rate_is_binomial(p):
    n = 200_000
    kept = D.keep(n, p, seed=7, offset=11)
    sd = np.sqrt(n * p * (1 - p))
    assert abs((n - kept.sum()) - n * p) < 6 * sd
    # streams of different offsets or seeds are not the same
    assert not np.array_equal(kept, D.keep(n, p, seed=7, offset=12))
    assert not np.array_equal(kept, D.keep(n, p, seed=8, offset=11))


def test_dropout_values():
    x = np.linspace(-3, 3, 1001, dtype=np.float32)
    y, m = D.dropout(x, 0.25, seed=3)
    scale = np.float32(1) / (np.float32(1) - np.float32(0.25))
    assert set(np.unique(m).tolist()) <= {0.0, float(scale)}
    assert np.array_equal(y, x * m)
    y0, m0 = D.dropout(x, 0.0, seed=3)
    assert np.array_equal(y0, x) and np.all(m0 == 1.0)
