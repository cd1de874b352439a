"""GPU parity of sporder_count_pillars and the quality metrics.

count_pillars is an integer count: equal to the oracle on every input,
including unsorted and duplicate columns, windows past the LDS capacity
(4096 nonzeros, sorted device-wide) and heights 1 and >= n.  The quality
metrics of P A P^T equal the oracle's (log_gap within 1e-12 relative).
"""

import numpy as np
import pytest
import torch

import oracle
from chunkedgreedy_amd import quality, synth

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).cuda()


def random_pattern(n, max_len, seed, hub=0):
    rng = np.random.default_rng(seed)
    lens = rng.integers(0, max_len, size=n)
    if hub:
        lens[n // 2] = hub
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(lens, out=ptr[1:])
    ind = rng.integers(0, n, size=int(ptr[-1]))  # unsorted, with duplicates
    return ptr.astype(np.int32), ind.astype(np.int32)


CASES = {
    "C1": synth.config1(61)[:2],
    "rmat12": synth.rmat(12, 16, 62)[:2],
    "stencil12": synth.stencil7(12, 63)[:2],
    "random_dups": random_pattern(5000, 20, 64),
    "hub_window": random_pattern(20000, 6, 65, hub=9000),
    "empty_rows": (np.array([0, 0, 3, 3, 5], np.int32), np.array([2, 2, 1, 0, 3], np.int32)),
}


@pytest.mark.parametrize("name", sorted(CASES))
@pytest.mark.parametrize("height", [1, 7, 16, 512, 1 << 20])
def test_count_pillars_exact(sporder, name, height):
    ptr, ind = CASES[name]
    print(f"[pillars] {name} h={height}", flush=True)
    assert sporder.count_pillars(dev(ptr), dev(ind), height) == oracle.count_pillars(
        ptr, ind, height)


def test_count_pillars_errors(sporder):
    with pytest.raises(ValueError):
        sporder.count_pillars(dev(np.array([0, 1])), dev(np.array([0])), 0)
    with pytest.raises(ValueError):
        sporder.count_pillars(dev(np.array([0])), dev(np.zeros(0)), 1)
    assert sporder.count_pillars(dev(np.zeros(5)), dev(np.zeros(0)), 4) == 0


@pytest.mark.parametrize("name", ["C1", "rmat12", "stencil12"])
def test_quality_metrics_of_reordered(sporder, name):
    ptr, ind = CASES[name]
    sym = synth.is_pattern_symmetric(ptr, ind)
    order = sporder.chunk_similarity_greedy(dev(ptr), dev(ind), is_symmetric=sym)
    got = quality.structure_metrics(dev(ptr), dev(ind), order)
    o = order.cpu().numpy().astype(np.int64)
    n = ptr.shape[0] - 1
    inv = np.empty(n, np.int64)
    inv[o] = np.arange(n)
    rows = np.repeat(np.arange(n), np.diff(ptr))
    want = oracle.quality_metrics(inv[rows], inv[ind.astype(np.int64)], n)
    for key in ("pillars", "tc_blocks", "bandwidth", "profile"):
        assert got[key] == want[key], key
    assert got["pillars_check"] == want["pillars"]
    assert got["log_gap"] == pytest.approx(want["log_gap"], rel=1e-12)
