"""Pins of the pillar count and the structural quality metrics (oracle).

Closed forms: the identity pattern (n pillars at height 1, n pillars for any
height since every column appears once, bandwidth 0, profile 0, log_gap 0),
a full band, a dense block and a single dense row; brute-force Python sets on
small random patterns with duplicate and unsorted columns.
"""

import numpy as np
import pytest

import oracle
from chunkedgreedy_amd import synth


def coo(ptr, ind):
    n = ptr.shape[0] - 1
    return np.repeat(np.arange(n), np.diff(ptr)), ind.astype(np.int64), n


def test_identity_closed_forms():
    n = 100
    ptr = np.arange(n + 1, dtype=np.int32)
    ind = np.arange(n, dtype=np.int32)
    for h in (1, 3, 16, 100, 1000):
        assert oracle.count_pillars(ptr, ind, h) == n
    m = oracle.quality_metrics(*coo(ptr, ind))
    assert m == {"pillars": n, "tc_blocks": sum((min(16, n - w) + 7) // 8
                                                 for w in range(0, n, 16)),
                 "bandwidth": 0, "profile": 0, "log_gap": 0.0}


def test_band_and_block_closed_forms():
    n, hw = 64, 2
    ptr, ind, _ = synth.band(n, hw)
    # Window of rows [a, a+h) touches columns [a-hw, a+h-1+hw] clipped to [0, n).
    for h in (1, 4, 16):
        want = sum(min(n, a + h + hw) - max(0, a - hw) for a in range(0, n, h))
        assert oracle.count_pillars(ptr, ind, h) == want
    m = oracle.quality_metrics(*coo(ptr, ind))
    assert m["bandwidth"] == hw
    assert m["profile"] == sum(min(i, hw) for i in range(n))
    # Dense 32 x 32 block: every window sees all 32 columns.
    d = 32
    ptr = np.arange(0, d * d + 1, d, dtype=np.int32)
    ind = np.tile(np.arange(d, dtype=np.int32), d)
    assert oracle.count_pillars(ptr, ind, 8) == 4 * d
    assert oracle.count_pillars(ptr, ind, 1) == d * d
    m = oracle.quality_metrics(*coo(ptr, ind))
    assert m["tc_blocks"] == 2 * (d // 8) and m["bandwidth"] == d - 1


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_pillars_brute_force_with_duplicates(seed):
    rng = np.random.default_rng(seed)
    n = 300
    lens = rng.integers(0, 12, size=n)
    ptr = np.zeros(n + 1, np.int32)
    np.cumsum(lens, out=ptr[1:])
    ind = rng.integers(0, n, size=ptr[-1]).astype(np.int32)  # unsorted, duplicates
    for h in (1, 5, 16, 300):
        want = len({(r // h, int(c)) for r in range(n) for c in ind[ptr[r]:ptr[r + 1]]})
        assert oracle.count_pillars(ptr, ind, h) == want


def test_reorder_bench_metrics_closed_forms():
    n, hw = 64, 3
    ptr, ind, _ = synth.band(n, hw)
    m = oracle.reorder_bench_metrics(ptr, ind, tc_h=16, tc_w=8)
    assert m["bandwidth"] == hw
    # Row i reaches i+hw (or the last column) and i-hw (or column 0).
    assert m["profile"] == sum(max(min(hw, i), min(hw, n - 1 - i)) for i in range(n))
    # Window of 16 rows starting at a sees columns [a-hw, a+15+hw] clipped.
    want_tc = sum(-(-(min(n, a + 16 + hw) - max(0, a - hw)) // 8) for a in range(0, n, 16))
    assert m["tc_num"] == want_tc
    assert m["tc_fill_rate"] == pytest.approx(ptr[-1] / (want_tc * 16 * 8))
    empty = oracle.reorder_bench_metrics(np.zeros(5, np.int32), np.zeros(0, np.int32))
    assert empty["tc_num"] == 0 and empty["bandwidth"] == 0
