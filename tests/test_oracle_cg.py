"""The oracle of sporder_chunk_greedy (cg): global sketch + per-chunk chain.

Pins:
  - with chunk_size >= n, cg and csg compute the same thing (one chunk of all
    rows for both the sketch and the chain), so their permutations and stats
    must agree;
  - the global table equals the chunked table with a chunk of n rows, and each
    row of it equals the sketch of the brute-force stream (every row of every
    column of the row, itself excluded, weight 2/(|r|+|s|));
  - cut_weight_fraction is 0 with a single chunk and 1 with chunks of one row
    (a row never lists itself), and equals a direct count in between (within
    1e-6: the total weight is summed per row in fp32, as the reference does);
  - the chain only follows in-chunk entries: every step either restarts at the
    lowest unvisited row or moves to the best unvisited in-chunk neighbour.
"""

import numpy as np
import pytest

import oracle
from chunkedgreedy_amd import synth

MATS = {
    "C1": synth.config1(31)[:2],
    "band300": synth.band(300)[:2],
    "rmat9": synth.rmat(9, 8, 32)[:2],
    "stencil7": synth.stencil7(7, 33)[:2],
}


@pytest.mark.parametrize("name", sorted(MATS))
def test_single_chunk_equals_csg(name):
    ptr, ind = MATS[name]
    n = ptr.shape[0] - 1
    sym = synth.is_pattern_symmetric(ptr, ind)
    o_cg, s_cg = oracle.chunk_greedy(ptr, ind, is_symmetric=sym, chunk_size=n)
    o_csg, s_csg = oracle.chunk_similarity_greedy(ptr, ind, is_symmetric=sym, chunk_size=n)
    assert np.array_equal(o_cg, o_csg)
    for key in ("k_used", "m_used", "zero_degree_rows", "chain_restarts"):
        assert s_cg[key] == s_csg[key]
    # The total weight is summed per row in fp32 (as the reference's
    # top-k statistics do), the in-chunk weight in fp64: equal up to rounding.
    assert s_cg["cut_weight_fraction"] <= 1e-6


@pytest.mark.parametrize("name", sorted(MATS))
def test_global_table_is_brute_force_sketch(name):
    ptr, ind = MATS[name]
    n = ptr.shape[0] - 1
    _, _, table = oracle.chunk_greedy(ptr, ind, chunk_size=64, k=8, oversampling=4.0,
                                      return_table=True)
    cptr, rind = oracle.csr2csc(ptr, ind)
    sizes = np.diff(ptr)
    for r in (0, n // 3, n - 1):
        keys, ws = [], []
        for c in ind[ptr[r]:ptr[r + 1]]:
            for s in rind[cptr[c]:cptr[c + 1]]:
                if s != r:
                    keys.append(s)
                    ws.append(np.float32(2.0) / np.float32(sizes[r] + sizes[s]))
        want = oracle.sketch_stream(32, 8, np.array(keys, np.int32), np.array(ws, np.float32))
        if sizes[r] == 0:
            want = np.zeros(8, np.uint64)
        assert np.array_equal(table[r], want), r


@pytest.mark.parametrize("name", sorted(MATS))
def test_cut_weight_fraction_closed_forms(name):
    ptr, ind = MATS[name]
    n = ptr.shape[0] - 1
    _, s1 = oracle.chunk_greedy(ptr, ind, chunk_size=1)
    if s1["avg_degree"] > 0:
        assert s1["cut_weight_fraction"] == 1.0  # no in-chunk entry at all
    _, s, table = oracle.chunk_greedy(ptr, ind, chunk_size=37, return_table=True)
    idx, w = oracle.unpack_table(table)
    tot = inside = 0.0
    for r in range(n):
        for j in range(table.shape[1]):
            if idx[r, j] < 0:
                break
            tot += float(w[r, j])
            if idx[r, j] // 37 == r // 37:
                inside += float(w[r, j])
    want = 1.0 - inside / tot if tot > 0 else 0.0
    assert abs(s["cut_weight_fraction"] - want) <= 1e-6


@pytest.mark.parametrize("name", sorted(MATS))
def test_chain_follows_in_chunk_entries(name):
    ptr, ind = MATS[name]
    n = ptr.shape[0] - 1
    C = 50
    order, stats, table = oracle.chunk_greedy(ptr, ind, chunk_size=C, return_table=True)
    idx, w = oracle.unpack_table(table)
    restarts = 0
    for start in range(0, n, C):
        end = min(start + C, n)
        seg = order[start:end]
        assert sorted(seg) == list(range(start, end))
        assert seg[0] == start
        seen = {seg[0]}
        for a, b in zip(seg[:-1], seg[1:]):
            cands = [(w[a, j], -idx[a, j]) for j in range(table.shape[1])
                     if idx[a, j] >= 0 and start <= idx[a, j] < end and idx[a, j] not in seen]
            if cands:
                assert b == -max(cands)[1]
            else:
                assert b == min(set(range(start, end)) - seen)
                restarts += 1
            seen.add(b)
    assert restarts == stats["chain_restarts"]
