"""The oracle's sketch + stream against independent computations.

* Stream: brute-force enumeration of the chunk-restricted candidate stream
  (for each column of r in CSR order, rows of that column ascending, inside
  r's chunk, not r) with scipy's transpose; alpha = fp32 2/(|r|+|s|).
* No-eviction closed form: when a row has at most M distinct candidates no
  slot is ever evicted, so slot = rank of first occurrence, weight = the
  repeated fp32 sum of the pair's alpha, and the output is the merge of the
  per-lane selection-sorted cells.  This is computed from counts and first
  occurrences, not by replaying the sketch.
"""

import numpy as np
import pytest
import scipy.sparse as sp

import oracle
from chunkedgreedy_amd import synth


def streams(ptr, ind, chunk):
    n = ptr.shape[0] - 1
    a = sp.csr_matrix((np.ones(ind.shape[0]), ind, ptr), shape=(n, n))
    csc = a.tocsc()
    csc.sort_indices()
    out = []
    for r in range(n):
        rs = int(ptr[r + 1] - ptr[r])
        cs = (r // chunk) * chunk
        ce = min(cs + chunk, n)
        items = []
        for p in range(ptr[r], ptr[r + 1]):
            c = ind[p]
            for s in csc.indices[csc.indptr[c]:csc.indptr[c + 1]]:
                if cs <= s < ce and s != r:
                    sz = int(ptr[s + 1] - ptr[s])
                    items.append((int(s), np.float32(2.0) / np.float32(rs + sz)))
        out.append(items)
    return out


def closed_form_row(items, m, k):
    """Expected top-k (index, weight) of a stream with <= m distinct keys."""
    cells = m // 32
    first = {}
    count = {}
    alpha = {}
    for key, a in items:
        if key not in first:
            first[key] = len(first)
            alpha[key] = a
        count[key] = count.get(key, 0) + 1
    assert len(first) <= m
    weight = {}
    for key, c in count.items():
        w = alpha[key]
        for _ in range(c - 1):
            w = np.float32(w + alpha[key])
        weight[key] = w
    lanes = [[] for _ in range(32)]
    for key, s in sorted(first.items(), key=lambda t: t[1]):
        lanes[s // cells].append((key, weight[key]))
    # Per-lane selection sort, descending, strict '>'.
    for lane in lanes:
        for i in range(len(lane) - 1):
            best = i
            for j in range(i + 1, len(lane)):
                if lane[j][1] > lane[best][1]:
                    best = j
            lane[i], lane[best] = lane[best], lane[i]
    out = []
    pos = [0] * 32
    while len(out) < k:
        heads = [(lanes[l][pos[l]][1] if pos[l] < len(lanes[l]) else -1.0, l) for l in range(32)]
        best_w = max(h[0] for h in heads)
        if best_w < 0:
            break
        lane = min(l for w, l in heads if w == best_w)
        out.append(lanes[lane][pos[lane]])
        pos[lane] += 1
    return out


def expect_table(ptr, ind, chunk, m, k):
    n = ptr.shape[0] - 1
    idx = np.full((n, k), -1, np.int32)
    w = np.zeros((n, k), np.float32)
    for r, items in enumerate(streams(ptr, ind, chunk)):
        for j, (key, wt) in enumerate(closed_form_row(items, m, k)):
            idx[r, j] = key
            w[r, j] = wt
    return idx, w


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("chunk", [7, 64, 10_000])
def test_no_eviction_closed_form_random(seed, chunk):
    rng = np.random.default_rng(seed)
    n = 200
    lens = rng.integers(0, 9, size=n)
    ptr = np.zeros(n + 1, np.int32)
    np.cumsum(lens, out=ptr[1:])
    ind = np.concatenate([np.sort(rng.choice(40, size=L, replace=False)) for L in lens]).astype(
        np.int32)
    k, ovs = 8, 64.0  # M = 512 >= any distinct count here: no eviction
    idx, w = expect_table(ptr, ind, chunk, 512, k)
    t = oracle.chunk_similarity_top_k(ptr, ind, k, chunk, ovs)
    oi, ow = oracle.unpack_table(t)
    assert np.array_equal(oi, idx)
    assert np.array_equal(ow.view(np.uint32), w.view(np.uint32))


@pytest.mark.parametrize("cells", [1, 2, 3, 4])
def test_no_eviction_closed_form_capacities(cells):
    """Small capacities (CELLS 1..4) where distinct candidates stay <= M."""
    ptr, ind, _ = synth.band(120, half_width=3)  # <= 12 distinct candidates per row
    m = 32 * cells
    k = 16
    idx, w = expect_table(ptr, ind, 120, m, k)
    t = oracle.chunk_similarity_top_k(ptr, ind, k, 120, m / k, is_symmetric=True)
    oi, ow = oracle.unpack_table(t)
    assert np.array_equal(oi, idx)
    assert np.array_equal(ow.view(np.uint32), w.view(np.uint32))


def test_symmetric_alias_equals_transpose():
    """For a symmetric pattern the CSR-as-CSC alias gives the transpose's table."""
    ptr, ind, _ = synth.stencil7(8, 3)
    a = oracle.chunk_similarity_top_k(ptr, ind, 16, 100, 4.0, is_symmetric=True)
    b = oracle.chunk_similarity_top_k(ptr, ind, 16, 100, 4.0, is_symmetric=False)
    assert np.array_equal(a, b)


def test_alpha_is_correctly_rounded_division():
    """alpha = fl32(2 / fl32(a + b)) for every size pair in a row."""
    ptr = np.array([0, 1, 3, 6, 10], np.int32)
    ind = np.array([0, 0, 1, 0, 1, 2, 0, 1, 2, 3], np.int32)
    t = oracle.chunk_similarity_top_k(ptr, ind, 4, 4, 8.0)
    idx, w = oracle.unpack_table(t)
    # Row 0 = {0} shares column 0 with rows 1 (|2|), 2 (|3|), 3 (|4|).
    expect = {1: np.float32(2) / np.float32(3), 2: np.float32(2) / np.float32(4),
              3: np.float32(2) / np.float32(5)}
    for j in range(3):
        assert w[0, j].view(np.uint32) == expect[idx[0, j]].view(np.uint32)
