"""The oracle's greedy chain against a brute-force nearest-neighbour chain
(textbook: follow the heaviest unvisited in-chunk neighbour, ties to the
smaller index; otherwise restart at the lowest unvisited row), and the
invariants of its output."""

import numpy as np
import pytest

import oracle
from chunkedgreedy_amd import synth


def brute_greedy(idx, w, chunk):
    n, k = idx.shape
    order = []
    restarts = 0
    links = 0
    for start in range(0, n, chunk):
        end = min(start + chunk, n)
        visited = set()
        cur = start
        while True:
            visited.add(cur)
            order.append(cur)
            cands = []
            for j in range(k):
                s = int(idx[cur, j])
                if s < 0:
                    break
                if start <= s < end and s not in visited:
                    cands.append((-float(w[cur, j]), s))
            if cands:
                cur = min(cands)[1]
                links += 1
                continue
            rest = [r for r in range(start, end) if r not in visited]
            if not rest:
                break
            restarts += 1
            cur = rest[0]
    return np.array(order, np.int32), restarts, links


def random_table(n, k, seed, in_chunk=None):
    rng = np.random.default_rng(seed)
    idx = np.full((n, k), -1, np.int32)
    w = np.zeros((n, k), np.float32)
    for r in range(n):
        d = rng.integers(0, k + 1)
        lo, hi = (0, n) if in_chunk is None else in_chunk(r)
        cand = rng.choice(np.arange(lo, hi), size=min(d, hi - lo), replace=False)
        ws = rng.choice(np.array([0.25, 0.5, 0.75, 1.0], np.float32), size=cand.size)
        o = np.lexsort((cand, -ws))
        idx[r, : cand.size] = cand[o]
        w[r, : cand.size] = ws[o]
    return idx, w


@pytest.mark.parametrize("chunk", [1, 5, 16, 100])
@pytest.mark.parametrize("seed", [0, 1])
def test_greedy_matches_brute_force(chunk, seed):
    n, k = 100, 6
    idx, w = random_table(n, k, seed)  # entries may leave the chunk: filtered
    order, counters = oracle.greedy(oracle.pack_table(idx, w), chunk)
    b_order, b_restarts, b_links = brute_greedy(idx, w, chunk)
    assert np.array_equal(order, b_order)
    assert counters["restarts"] == b_restarts
    assert counters["links"] == b_links


def test_greedy_invariants_on_pipeline_output():
    ptr, ind, _ = synth.config1(3)
    order, stats, table = oracle.chunk_similarity_greedy(ptr, ind, return_table=True)
    n = ptr.shape[0] - 1
    C = stats["chunk_size_used"]
    idx, w = oracle.unpack_table(table)
    for start in range(0, n, C):
        end = min(start + C, n)
        seg = order[start:end]
        assert np.array_equal(np.sort(seg), np.arange(start, end))  # permutation of chunk
        assert seg[0] == start                                        # chain starts at start
    # Every step follows a top-k edge or restarts at the lowest unvisited row.
    b_order, b_restarts, _ = brute_greedy(idx, w, C)
    assert np.array_equal(order, b_order)
    assert stats["chain_restarts"] == b_restarts


def test_stats_closed_forms():
    ptr, ind, _ = synth.band(500)
    order, stats, table = oracle.chunk_similarity_greedy(ptr, ind, is_symmetric=True,
                                                         return_table=True)
    idx, w = oracle.unpack_table(table)
    deg = (idx >= 0).sum(axis=1)
    assert stats["zero_degree_rows"] == int((deg == 0).sum())
    assert stats["avg_degree"] == pytest.approx(deg.sum() / 500, rel=1e-12)
    assert stats["avg_edge_weight"] == pytest.approx(
        float(w[idx >= 0].astype(np.float64).sum()) / deg.sum(), rel=1e-6)
    # The band chain follows i -> i+1 inside each chunk: no restarts.
    assert stats["chain_restarts"] == 0
    assert np.array_equal(order, np.arange(500))
