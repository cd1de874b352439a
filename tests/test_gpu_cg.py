"""GPU parity of sporder_chunk_greedy (sporder-cg): HIP library vs the oracle.

The permutation and the integer statistics are bit-exact; the double
statistics within 1e-9 relative (atomic sums), cut_weight_fraction within 1e-6
(the total weight is summed per row in fp32, as the reference does, so its low
bits depend on the order of rows).
"""

import numpy as np
import pytest
import torch

import oracle
from chunkedgreedy_amd import synth

pytestmark = pytest.mark.gpu


def dev_csr(ptr, ind, dev="cuda:0"):
    return (torch.from_numpy(np.ascontiguousarray(ptr, np.int32)).to(dev),
            torch.from_numpy(np.ascontiguousarray(ind, np.int32)).to(dev))


MATS = {
    "band1000": synth.band(1000)[:2],
    "C1": synth.config1(41)[:2],
    "planted64k": synth.planted(1 << 16, 1024, 16, 42)[:2],
    "stencil20": synth.stencil7(20, 43)[:2],
    "stencil20_ordered": synth.stencil7(20, 43, scramble=False)[:2],
    "rmat11": synth.rmat(11, 16, 44)[:2],
    "chunglu5k": synth.chung_lu(5000, 2.1, 16, 45)[:2],
}


@pytest.mark.parametrize("name", sorted(MATS))
@pytest.mark.parametrize("k,ovs,chunk", [(0, 0.0, 0), (8, 2.0, 64), (24, 4.0, 4096),
                                         (16, 4.0, 5000), (8, 4.0, 1)])
def test_cg_permutation_bit_exact(sporder, name, k, ovs, chunk):
    ptr, ind = MATS[name]
    sym = synth.is_pattern_symmetric(ptr, ind)
    print(f"[cg] {name} k={k} ovs={ovs} chunk={chunk}", flush=True)
    dptr, dind = dev_csr(ptr, ind)
    order, timing, stats = sporder.chunk_greedy(dptr, dind, is_symmetric=sym, k=k,
                                                oversampling=ovs, chunk_size=chunk,
                                                with_timing=True, with_stats=True)
    o_order, o_stats = oracle.chunk_greedy(ptr, ind, is_symmetric=sym, k=k, oversampling=ovs,
                                           chunk_size=chunk)
    assert np.array_equal(order.cpu().numpy(), o_order)
    for key in ("k_used", "m_used", "zero_degree_rows", "chunk_size_used", "chain_restarts"):
        assert stats[key] == o_stats[key], key
    for key in ("avg_degree", "avg_edge_weight", "avg_followed_weight"):
        assert stats[key] == pytest.approx(o_stats[key], rel=1e-9, abs=1e-12), key
    assert abs(stats["cut_weight_fraction"] - o_stats["cut_weight_fraction"]) <= 1e-6
    assert set(timing) == {"wall_ms", "csr2csc_ms", "similarity_ms", "chunk_greedy_ms"}
    assert timing["wall_ms"] >= timing["chunk_greedy_ms"] >= 0.0


@pytest.mark.parametrize("k,ovs", [(512, 1.0), (257, 1.5)])
def test_cg_large_k_wide_chunks(sporder, k, ovs):
    """Chain chunks of 4096 rows with k past 256 (slices past 2^20 table
    entries) read the table in global memory: bit-exact permutation."""
    ptr, ind = MATS["chunglu5k"]
    sym = synth.is_pattern_symmetric(ptr, ind)
    dptr, dind = dev_csr(ptr, ind)
    order, stats = sporder.chunk_greedy(dptr, dind, is_symmetric=sym, k=k, oversampling=ovs,
                                        chunk_size=4096, with_stats=True)
    o_order, o_stats = oracle.chunk_greedy(ptr, ind, is_symmetric=sym, k=k, oversampling=ovs,
                                           chunk_size=4096)
    assert np.array_equal(order.cpu().numpy(), o_order)
    assert stats["chain_restarts"] == o_stats["chain_restarts"]


def test_cg_single_chunk_equals_csg(sporder):
    ptr, ind = MATS["C1"]
    n = ptr.shape[0] - 1
    dptr, dind = dev_csr(ptr, ind)
    a = sporder.chunk_greedy(dptr, dind, chunk_size=n)
    b = sporder.chunk_similarity_greedy(dptr, dind, chunk_size=n)
    assert torch.equal(a, b)


def test_cg_return_shapes_and_edges(sporder):
    ptr, ind = MATS["C1"]
    dptr, dind = dev_csr(ptr, ind)
    o = sporder.chunk_greedy(dptr, dind)
    assert isinstance(o, torch.Tensor) and o.dtype == torch.int32 and o.shape == (20000,)
    o2, s = sporder.chunk_greedy(dptr, dind, with_stats=True)
    assert torch.equal(o, o2) and "cut_weight_fraction" in s and s["k_used"] == 16
    cases = [
        (np.array([0, 0], np.int32), np.zeros(0, np.int32)),
        (np.array([0, 1], np.int32), np.array([0], np.int32)),
        (np.array([0, 0, 2, 2, 4, 4], np.int32), np.array([1, 3, 1, 3], np.int32)),
        (np.zeros(101, np.int32), np.zeros(0, np.int32)),
    ]
    for p, i in cases:
        for chunk in (0, 1, 3):
            g = sporder.chunk_greedy(*dev_csr(p, i), chunk_size=chunk).cpu().numpy()
            want, _ = oracle.chunk_greedy(p, i, chunk_size=chunk)
            assert np.array_equal(g, want), (p, i, chunk)
    with pytest.raises(ValueError):
        sporder.chunk_greedy(torch.zeros(1, dtype=torch.int32, device="cuda"),
                             torch.zeros(0, dtype=torch.int32, device="cuda"))


def small_blocks(n, block, deg, seed):
    """Symmetric pattern with columns inside diagonal blocks of `block` rows:
    each row is similar to its block-mates only."""
    rng = np.random.default_rng(seed)
    rows = np.repeat(np.arange(n), deg)
    cols = np.minimum((rows // block) * block + rng.integers(0, block, size=n * deg), n - 1)
    rows, cols = np.concatenate([rows, cols]), np.concatenate([cols, rows])
    keys = np.unique(rows.astype(np.int64) * n + cols)
    r, c = keys // n, keys % n
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(np.bincount(r, minlength=n), out=ptr[1:])
    return ptr.astype(np.int32), c.astype(np.int32)


def test_cg_sparse_table_many_chunks(sporder):
    """Global table with two or three valid entries per row and chain chunks
    (64 rows) that cut blocks of 3: many chunks, so the chain stages each
    row's valid prefix from the sketch's counts, including rows whose entries
    fall partly outside their chunk.  Bit-exact permutation and restarts."""
    ptr, ind = small_blocks(60000, 3, 3, 61)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert 60000 // 64 > 2 * cus
    dptr, dind = dev_csr(ptr, ind)
    order, stats = sporder.chunk_greedy(dptr, dind, is_symmetric=True, k=16, oversampling=4.0,
                                        chunk_size=64, with_stats=True)
    o_order, o_stats = oracle.chunk_greedy(ptr, ind, is_symmetric=True, k=16, oversampling=4.0,
                                           chunk_size=64)
    assert o_stats["avg_degree"] < 4.0
    assert np.array_equal(order.cpu().numpy(), o_order)
    assert stats["chain_restarts"] == o_stats["chain_restarts"]
