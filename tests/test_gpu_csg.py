"""GPU parity of the Chunked Greedy path: HIP library vs the CPU oracle.

Bit-exact comparisons (integer and index work, and the fp32 sketch weights,
whose accumulation order the reference fixes).  Inputs are seeded synthetic
matrices at sizes the oracle finishes in seconds, plus the full headline
configuration (C2) where the oracle is still fast.
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


def weight_bits(w):
    return np.ascontiguousarray(w, np.float32).view(np.uint32)


def small_matrices():
    out = {
        "band1000": synth.band(1000)[:2],
        "C1": synth.config1(11)[:2],
        "planted64k": synth.planted(1 << 16, 1024, 16, 12)[:2],
        "stencil20": synth.stencil7(20, 13)[:2],
        "stencil20_ordered": synth.stencil7(20, 13, scramble=False)[:2],
        "rmat13": synth.rmat(13, 16, 14)[:2],
        "rmat11": synth.rmat(11, 16, 16)[:2],
        "chunglu20k": synth.chung_lu(20000, 2.1, 25, 15)[:2],
    }
    return out


MATS = small_matrices()


def check_table(sp, ptr, ind, k, ovs, chunk, sym):
    print(f"[table] n={ptr.shape[0]-1} nnz={ind.shape[0]} k={k} ovs={ovs} chunk={chunk} "
          f"sym={sym}", flush=True)
    dptr, dind = dev_csr(ptr, ind)
    gi, gw = sp.chunk_similarity_top_k(dptr, dind, k=k, oversampling=ovs, chunk_size=chunk,
                                       is_symmetric=sym)
    t = oracle.chunk_similarity_top_k(ptr, ind, k, chunk, ovs, is_symmetric=sym)
    oi, ow = oracle.unpack_table(t)
    gi = gi.cpu().numpy()
    gw = gw.cpu().numpy()
    mism = np.nonzero((gi != oi).any(axis=1) | (weight_bits(gw) != weight_bits(ow)).any(axis=1))[0]
    assert mism.size == 0, (f"{mism.size} rows differ; first row {mism[0]}: gpu "
                            f"{gi[mism[0]]} {gw[mism[0]]} oracle {oi[mism[0]]} {ow[mism[0]]}")
    return oi, ow


@pytest.mark.parametrize("name", sorted(MATS))
@pytest.mark.parametrize("k,ovs,chunk", [(16, 4.0, 1024), (8, 4.0, 256), (16, 1.0, 4096),
                                         (24, 4.0, 1024), (5, 3.5, 333), (32, 16.0, 2048)])
def test_chunk_table_bit_exact(sporder, name, k, ovs, chunk):
    ptr, ind = MATS[name]
    sym = synth.is_pattern_symmetric(ptr, ind)
    check_table(sporder, ptr, ind, k, ovs, chunk, sym)


@pytest.mark.parametrize("name", ["rmat13", "chunglu20k", "C1"])
def test_chunk_table_nonsymmetric_path(sporder, name):
    """Symmetric patterns through the transpose path give the same table."""
    ptr, ind = MATS[name]
    check_table(sporder, ptr, ind, 16, 4.0, 1024, False)


@pytest.mark.parametrize("ovs", [1.0, 2.0, 4.0, 8.0, 16.0, 32.0])
def test_global_sketch_all_capacities(sporder, ovs):
    """Sketch capacities 32..512 (CELLS 1..16) on a hub-heavy graph, one chunk
    spanning all rows (heavy eviction)."""
    ptr, ind = MATS["rmat11"]
    n = ptr.shape[0] - 1
    check_table(sporder, ptr, ind, 16, ovs, n, True)


@pytest.mark.parametrize("k,ovs", [(3, 32.0), (7, 13.0), (10, 10.0), (48, 2.0), (100, 5.0),
                                   (256, 2.0)])
def test_global_sketch_odd_capacities(sporder, k, ovs):
    ptr, ind = MATS["chunglu20k"]
    n = ptr.shape[0] - 1
    check_table(sporder, ptr, ind, k, ovs, n, True)


def test_band_known_answer(sporder):
    """Band |i-j|<=2 (the reference smoke matrix), k=8, ovs=4 -> M=32: row 0's
    neighbours are 1,2,3,4 with weights 3 sequential adds of fl(2/7), 0.75,
    0.5, 0.25 (golden vector)."""
    ptr, ind = MATS["band1000"]
    dptr, dind = dev_csr(ptr, ind)
    idx, wgt = sporder.similarity_graph(dptr, dind, is_symmetric=True, k=8, oversampling=4.0)
    idx = idx.cpu().numpy()
    wgt = wgt.cpu().numpy()
    assert idx[0].tolist() == [1, 2, 3, 4, -1, -1, -1, -1]
    assert weight_bits(wgt[0]).tolist() == [0x3F5B6DB8, 0x3F400000, 0x3F000000, 0x3E800000,
                                            0, 0, 0, 0]
    assert 0 < idx[0, 0] < 1000


@pytest.mark.parametrize("name", sorted(MATS))
@pytest.mark.parametrize("k,ovs,chunk", [(0, 0.0, 0), (16, 4.0, 256), (24, 2.0, 5000),
                                         (8, 4.0, 1)])
def test_csg_permutation_bit_exact(sporder, name, k, ovs, chunk):
    ptr, ind = MATS[name]
    sym = synth.is_pattern_symmetric(ptr, ind)
    print(f"[csg] {name} k={k} ovs={ovs} chunk={chunk}", flush=True)
    dptr, dind = dev_csr(ptr, ind)
    order, timing, stats = sporder.chunk_similarity_greedy(
        dptr, dind, is_symmetric=sym, k=k, oversampling=ovs, chunk_size=chunk,
        with_timing=True, with_stats=True)
    o_order, o_stats = oracle.chunk_similarity_greedy(ptr, ind, is_symmetric=sym, k=k,
                                                      oversampling=ovs, chunk_size=chunk)
    g = order.cpu().numpy()
    assert np.array_equal(g, o_order)
    for key in ("k_used", "m_used", "zero_degree_rows", "chunk_size_used", "chain_restarts"):
        assert stats[key] == o_stats[key], key
    for key in ("avg_degree", "avg_edge_weight", "avg_followed_weight"):
        # Doubles summed with atomics: order-dependent low bits.
        assert stats[key] == pytest.approx(o_stats[key], rel=1e-9, abs=1e-12), key
    assert set(timing) == {"wall_ms", "csr2csc_ms", "similarity_ms", "chunk_greedy_ms"}
    assert timing["wall_ms"] >= timing["chunk_greedy_ms"] >= 0.0


@pytest.mark.parametrize("k,ovs", [(512, 1.0), (257, 1.5), (256, 2.0)])
def test_csg_large_k_wide_chunks(sporder, k, ovs):
    """Chunks of 4096 rows with k past 256: the slice holds more than 2^20
    table entries, which the LDS-compacted chain cannot index, so the chain
    reads the table in global memory; k = 256 is the largest that compacts.
    Permutation and restart count bit-exact."""
    for name in ("chunglu20k", "rmat13"):
        ptr, ind = MATS[name]
        sym = synth.is_pattern_symmetric(ptr, ind)
        print(f"[csg-large-k] {name} k={k} ovs={ovs}", flush=True)
        dptr, dind = dev_csr(ptr, ind)
        order, stats = sporder.chunk_similarity_greedy(dptr, dind, is_symmetric=sym, k=k,
                                                       oversampling=ovs, chunk_size=4096,
                                                       with_stats=True)
        o_order, o_stats = oracle.chunk_similarity_greedy(ptr, ind, is_symmetric=sym, k=k,
                                                          oversampling=ovs, chunk_size=4096)
        assert np.array_equal(order.cpu().numpy(), o_order)
        assert stats["k_used"] == k and stats["chain_restarts"] == o_stats["chain_restarts"]


def test_csg_return_shapes(sporder):
    ptr, ind = MATS["C1"]
    dptr, dind = dev_csr(ptr, ind)
    o = sporder.chunk_similarity_greedy(dptr, dind)
    assert isinstance(o, torch.Tensor) and o.dtype == torch.int32 and o.shape == (20000,)
    o2, t = sporder.chunk_similarity_greedy(dptr, dind, with_timing=True)
    assert torch.equal(o, o2) and isinstance(t, dict)
    o3, s = sporder.chunk_similarity_greedy(dptr, dind, with_stats=True)
    assert torch.equal(o, o3) and s["k_used"] == 16 and s["m_used"] == 64
    o4, t4, s4 = sporder.chunk_similarity_greedy(dptr, dind, with_timing=True, with_stats=True)
    assert torch.equal(o, o4)


def test_csg_edge_cases(sporder):
    # Empty rows, a single row, no nonzeros at all, chunk larger than n.
    cases = [
        (np.array([0, 0], np.int32), np.zeros(0, np.int32)),
        (np.array([0, 1], np.int32), np.array([0], np.int32)),
        (np.array([0, 0, 2, 2, 4, 4], np.int32), np.array([1, 3, 1, 3], np.int32)),
        (np.zeros(101, np.int32), np.zeros(0, np.int32)),
    ]
    for ptr, ind in cases:
        for chunk in (0, 1, 3, 1000):
            dptr, dind = dev_csr(ptr, ind)
            g = sporder.chunk_similarity_greedy(dptr, dind, chunk_size=chunk).cpu().numpy()
            o, _ = oracle.chunk_similarity_greedy(ptr, ind, chunk_size=chunk)
            assert np.array_equal(g, o), (ptr, ind, chunk)


def test_csg_rejects_bad_sizes(sporder):
    with pytest.raises(ValueError):
        sporder.chunk_similarity_greedy(torch.zeros(1, dtype=torch.int32, device="cuda"),
                                        torch.zeros(0, dtype=torch.int32, device="cuda"))
    with pytest.raises(TypeError):
        sporder.chunk_similarity_greedy(torch.zeros(3, dtype=torch.int64, device="cuda"),
                                        torch.zeros(0, dtype=torch.int32, device="cuda"))


def test_csg_headline_config_bit_exact(sporder):
    """Full C2 (n = 2^20, 16 nnz/row, seed 2: the bench's matrix): csg
    permutation and table, then the symmetric permutation apply with values
    (P A P^T) and the reordered SpMM at N = 32 and N = 128 (B = torch.randn,
    seed 42, as the bench draws it), all bit-exact against the oracle."""
    ptr, ind, val = synth.config2(seed=2)
    print("[csg] C2 full", flush=True)
    dptr, dind = dev_csr(ptr, ind)
    order, stats = sporder.chunk_similarity_greedy(dptr, dind, with_stats=True)
    o_order, o_stats, o_table = oracle.chunk_similarity_greedy(ptr, ind, return_table=True)
    assert np.array_equal(order.cpu().numpy(), o_order)
    assert stats["chain_restarts"] == o_stats["chain_restarts"]
    assert np.array_equal(sporder.chunk_similarity_greedy(dptr, dind).cpu().numpy(), o_order)
    gi, gw = sporder.chunk_similarity_top_k(dptr, dind, k=16, oversampling=4.0, chunk_size=1024)
    oi, ow = oracle.unpack_table(o_table)
    assert np.array_equal(gi.cpu().numpy(), oi)
    assert np.array_equal(weight_bits(gw.cpu().numpy()), weight_bits(ow))
    # Size-independent property: each chunk's slice is a permutation of itself.
    n = ptr.shape[0] - 1
    g = order.cpu().numpy().reshape(-1, 1024)
    assert np.array_equal(np.sort(g, axis=1), np.arange(n).reshape(-1, 1024))

    dval = torch.from_numpy(val).to("cuda:0")
    p2, i2, v2 = sporder.reorder(dptr, dind, order, val=dval, symmetric=True)
    op, oi, ov = oracle.reorder(ptr, ind, o_order, val=val, symmetric=True)
    assert np.array_equal(p2.cpu().numpy(), op)
    assert np.array_equal(i2.cpu().numpy(), oi)
    assert np.array_equal(v2.cpu().numpy().view(np.uint32), ov.view(np.uint32))
    for N in (32, 128):
        gen = torch.Generator(device="cuda:0").manual_seed(42)
        B = torch.randn((n, N), generator=gen, dtype=torch.float32, device="cuda:0")
        C, _ = sporder.spmm_csr(p2, i2, v2, B)
        ref = oracle.spmm_csr(op, oi, ov, B.cpu().numpy())
        print(f"[csg] C2 full spmm N={N}", flush=True)
        assert np.array_equal(C.cpu().numpy().view(np.uint32), ref.view(np.uint32)), N


@pytest.mark.parametrize("name", ["C3", "C4", "C5"])
def test_full_config_bit_exact(sporder, name):
    """Full-size power-law and mesh configurations (C3 R-MAT scale 22, C4 160^3
    stencil, C5 Chung-Lu with 613K-entry hubs): csg permutation and chain
    restarts, the permutation apply with values, and the reordered SpMM at
    every width the configuration names, all bit-exact against the oracle."""
    import time

    gen = {"C3": synth.config3, "C4": synth.config4, "C5": synth.config5}[name]
    t0 = time.time()
    ptr, ind, val = gen()
    sym = synth.is_pattern_symmetric(ptr, ind)
    print(f"[full] {name} n={ptr.shape[0] - 1} nnz={ind.shape[0]} ({time.time() - t0:.1f}s)",
          flush=True)
    dptr, dind = dev_csr(ptr, ind)
    order, stats = sporder.chunk_similarity_greedy(dptr, dind, is_symmetric=sym,
                                                   with_stats=True)
    t0 = time.time()
    o_order, o_stats = oracle.chunk_similarity_greedy(ptr, ind, is_symmetric=sym)
    print(f"[full] {name} oracle csg {time.time() - t0:.1f}s", flush=True)
    assert np.array_equal(order.cpu().numpy(), o_order)
    assert stats["chain_restarts"] == o_stats["chain_restarts"]
    assert stats["zero_degree_rows"] == o_stats["zero_degree_rows"]
    # Without statistics the chain runs without its counters: same permutation.
    assert np.array_equal(
        sporder.chunk_similarity_greedy(dptr, dind, is_symmetric=sym).cpu().numpy(), o_order)

    dval = torch.from_numpy(val).to("cuda:0")
    p2, i2, v2 = sporder.reorder(dptr, dind, order, val=dval, symmetric=True)
    t0 = time.time()
    op, oi, ov = oracle.reorder(ptr, ind, o_order, val=val, symmetric=True)
    print(f"[full] {name} oracle reorder {time.time() - t0:.1f}s", flush=True)
    assert np.array_equal(p2.cpu().numpy(), op)
    assert np.array_equal(i2.cpu().numpy(), oi)
    assert np.array_equal(v2.cpu().numpy().view(np.uint32), ov.view(np.uint32))

    widths = {"C3": (32, 64, 256), "C4": (16, 32, 64, 128, 256), "C5": (128,)}[name]
    n = ptr.shape[0] - 1
    for N in widths:
        B = np.random.default_rng(42).standard_normal((n, N)).astype(np.float32)
        C, _ = sporder.spmm_csr(p2, i2, v2, torch.from_numpy(B).to("cuda:0"))
        t0 = time.time()
        ref = oracle.spmm_csr(op, oi, ov, B)
        print(f"[full] {name} oracle spmm N={N} {time.time() - t0:.1f}s", flush=True)
        assert np.array_equal(C.cpu().numpy().view(np.uint32), ref.view(np.uint32)), N
        del B, C, ref


@pytest.mark.parametrize("k,chunk", [(96, 1024), (72, 1024), (128, 2048), (96, 512)])
def test_csg_rows_past_one_wave(sporder, k, chunk):
    """Chunks whose rows hold about 70 and about 40 in-chunk entries
    (synth.dense_groups): the chain's read-ahead steps run in assembly for the
    shorter rows and hand the longer ones (more than 64 entries, past one
    wave's lanes) to the compiled scan; 2048-row chunks (64 bitmap words)
    are the largest the assembly steps take.  Permutation, restarts and
    followed weight bit-exact against the oracle."""
    ptr, ind, _ = synth.dense_groups()
    sym = synth.is_pattern_symmetric(ptr, ind)
    print(f"[dense-groups] k={k} chunk={chunk}", flush=True)
    dptr, dind = dev_csr(ptr, ind)
    for with_stats in (True, False):
        got = sporder.chunk_similarity_greedy(dptr, dind, is_symmetric=sym, k=k,
                                              chunk_size=chunk, with_stats=with_stats)
        order, stats = got if with_stats else (got, None)
        o_order, o_stats = oracle.chunk_similarity_greedy(ptr, ind, is_symmetric=sym, k=k,
                                                          chunk_size=chunk)
        assert np.array_equal(order.cpu().numpy(), o_order), with_stats
        if stats is not None:
            assert stats["chain_restarts"] == o_stats["chain_restarts"]
            assert stats["avg_followed_weight"] == pytest.approx(
                o_stats["avg_followed_weight"], rel=1e-9, abs=1e-12)


@pytest.mark.parametrize("name", ["C2r", "C4n", "RGG20"])
def test_locality_inputs_bit_exact(sporder, name):
    """The inputs with in-chunk locality at full size (C2 in planted row order,
    the 160^3 stencil in grid order, a random geometric graph): their chains
    take long links through rows of several in-chunk entries (the read-ahead
    walk, 64-bit and packed 16-bit entries).  csg permutation and restarts,
    with and without statistics, bit-exact against the oracle."""
    import time

    ptr, ind, _ = synth.LOCALITY[name]()
    sym = synth.is_pattern_symmetric(ptr, ind)
    print(f"[locality] {name} n={ptr.shape[0] - 1} nnz={ind.shape[0]}", flush=True)
    dptr, dind = dev_csr(ptr, ind)
    order, stats = sporder.chunk_similarity_greedy(dptr, dind, is_symmetric=sym,
                                                   with_stats=True)
    t0 = time.time()
    o_order, o_stats = oracle.chunk_similarity_greedy(ptr, ind, is_symmetric=sym)
    print(f"[locality] {name} oracle csg {time.time() - t0:.1f}s", flush=True)
    assert np.array_equal(order.cpu().numpy(), o_order)
    assert stats["chain_restarts"] == o_stats["chain_restarts"]
    # Per-chunk float sums of the followed weights, added as doubles with atomics.
    assert stats["avg_followed_weight"] == pytest.approx(o_stats["avg_followed_weight"],
                                                         rel=1e-9, abs=1e-12)
    assert np.array_equal(
        sporder.chunk_similarity_greedy(dptr, dind, is_symmetric=sym).cpu().numpy(), o_order)


GOLDEN = __import__("json").loads(
    (__import__("pathlib").Path(__file__).parent / "golden" / "sketch_cases.json").read_text())


@pytest.mark.parametrize("case", GOLDEN["csr_cases"], ids=lambda c: c["name"])
def test_golden_csr_cases(sporder, case):
    """Hand-worked eviction / Dice-weight cases (tests/golden/make_golden.py)."""
    ptr = np.array(case["ptr"], np.int32)
    ind = np.array(case["ind"], np.int32)
    dptr, dind = dev_csr(ptr, ind)
    k = case["k"]
    for chk in case["checks"]:
        gi, gw = sporder.chunk_similarity_top_k(dptr, dind, k=k, oversampling=case["oversampling"],
                                                chunk_size=chk["chunk"])
        r = chk["row"]
        exp_idx = [e[0] for e in chk["expected"]] + [-1] * (k - len(chk["expected"]))
        exp_bits = chk["expected_bits"] + [0] * (k - len(chk["expected"]))
        assert gi.cpu().numpy()[r].tolist() == exp_idx, chk
        assert weight_bits(gw.cpu().numpy()[r]).tolist() == exp_bits, chk


def dense_random(n, deg, seed, symmetric):
    rng = np.random.default_rng(seed)
    rows = np.repeat(np.arange(n), deg)
    cols = rng.integers(0, n, size=n * deg)
    if symmetric:
        rows, cols = np.concatenate([rows, cols]), np.concatenate([cols, rows])
    keys = np.unique(rows.astype(np.int64) * n + cols)
    r, c = keys // n, keys % n
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(np.bincount(r, minlength=n), out=ptr[1:])
    return ptr.astype(np.int32), c.astype(np.int32)


@pytest.mark.parametrize("symmetric", [False, True])
@pytest.mark.parametrize("chunk", [4096, 1500])
def test_overflow_chunks_take_global_path(sporder, symmetric, chunk):
    """Chunks with more nonzeros than the LDS key capacity (32768) go to the
    global-CSC kernel; the result is still bit-exact."""
    ptr, ind = dense_random(12000, 20 if symmetric else 40, 31, symmetric)
    assert synth.is_pattern_symmetric(ptr, ind) == symmetric
    check_table(sporder, ptr, ind, 16, 4.0, chunk, symmetric)
    dptr, dind = dev_csr(ptr, ind)
    g = sporder.chunk_similarity_greedy(dptr, dind, is_symmetric=symmetric, chunk_size=chunk)
    o, _ = oracle.chunk_similarity_greedy(ptr, ind, is_symmetric=symmetric, chunk_size=chunk)
    assert np.array_equal(g.cpu().numpy(), o)


def hub_rows_matrix(n, base_deg, hubs, seed, symmetric):
    """Random rows of base_deg columns plus hub rows {row: degree} whose
    columns are mostly distinct (empty runs within the chunk) with a few
    shared with their chunk's rows; hub rows start at unaligned offsets."""
    rng = np.random.default_rng(seed)
    rows = [np.repeat(np.arange(n), base_deg)]
    cols = [rng.integers(0, n, size=n * base_deg)]
    for r, d in hubs.items():
        rows.append(np.full(d, r))
        cols.append(rng.choice(n, size=d, replace=False))
    rows, cols = np.concatenate(rows), np.concatenate(cols)
    if symmetric:
        rows, cols = np.concatenate([rows, cols]), np.concatenate([cols, rows])
    keys = np.unique(rows.astype(np.int64) * n + cols)
    r, c = keys // n, keys % n
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(np.bincount(r, minlength=n), out=ptr[1:])
    return ptr.astype(np.int32), c.astype(np.int32)


@pytest.mark.parametrize("symmetric", [False, True])
@pytest.mark.parametrize("chunk", [1024, 1500])
def test_global_path_high_degree_rows(sporder, symmetric, chunk):
    """Global-path rows of at least 2048 nonzeros visit only the 64-nonzero
    blocks the run search marked as holding a non-empty run; chunks past the
    LDS capacity holding rows of 2047, 2048 and 2049 up to 15,000 nonzeros
    (many empty runs, unaligned block offsets) and ordinary chunks beside them
    give the oracle's table and permutation bit for bit."""
    hubs = {5: 2047, 6: 2048, 700: 2049, 701: 9000, 702: 9000, 703: 9000, 1031: 5000,
            1032: 15000, 1033: 15000, 3003: 12000, 3004: 12000, 3005: 12000, 9001: 3333,
            9002: 2500}
    ptr, ind = hub_rows_matrix(20000, 3, hubs, 41, symmetric)
    assert synth.is_pattern_symmetric(ptr, ind) == symmetric
    check_table(sporder, ptr, ind, 16, 4.0, chunk, symmetric)
    dptr, dind = dev_csr(ptr, ind)
    g = sporder.chunk_similarity_greedy(dptr, dind, is_symmetric=symmetric, chunk_size=chunk)
    o, _ = oracle.chunk_similarity_greedy(ptr, ind, is_symmetric=symmetric, chunk_size=chunk)
    assert np.array_equal(g.cpu().numpy(), o)


def test_tier2_split_symmetric(sporder):
    """On a symmetric pattern tier 2 keeps chunks of at most 28,672 nonzeros
    and the larger ones, up to its 32,768 capacity, go to the global path,
    which runs beside it; chunks on both sides of the split (no tier-1 chunk
    here) give the oracle's table and permutation bit for bit."""
    n, chunk = 6144, 1024
    degs = [10, 13, 16, 12, 17, 9]
    rng = np.random.default_rng(43)
    rows = np.concatenate([np.repeat(np.arange(q * chunk, (q + 1) * chunk), d)
                           for q, d in enumerate(degs)])
    cols = rng.integers(0, n, size=rows.size)
    rows, cols = np.concatenate([rows, cols]), np.concatenate([cols, rows])
    keys = np.unique(rows.astype(np.int64) * n + cols)
    r, c = keys // n, keys % n
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(np.bincount(r, minlength=n), out=ptr[1:])
    ptr, ind = ptr.astype(np.int32), c.astype(np.int32)
    E = ptr[chunk::chunk] - ptr[:-1:chunk]
    assert ((E > 16384) & (E <= 28672)).any() and ((E > 28672) & (E <= 32768)).any()
    check_table(sporder, ptr, ind, 16, 4.0, chunk, True)
    dptr, dind = dev_csr(ptr, ind)
    g = sporder.chunk_similarity_greedy(dptr, dind, is_symmetric=True, chunk_size=chunk)
    o, _ = oracle.chunk_similarity_greedy(ptr, ind, is_symmetric=True, chunk_size=chunk)
    assert np.array_equal(g.cpu().numpy(), o)


def hub_matrix(n, deg, hubs, seed, symmetric):
    """Random rows of `deg` columns plus hub rows {row: nonzeros}."""
    rng = np.random.default_rng(seed)
    rows = [np.repeat(np.arange(n), deg)]
    cols = [rng.integers(0, n, size=n * deg)]
    for r, d in hubs.items():
        rows.append(np.full(d, r))
        cols.append(rng.choice(n, size=d, replace=False))
    rows, cols = np.concatenate(rows), np.concatenate(cols)
    if symmetric:
        rows, cols = np.concatenate([rows, cols]), np.concatenate([cols, rows])
    keys = np.unique(rows.astype(np.int64) * n + cols)
    r, c = keys // n, keys % n
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(np.bincount(r, minlength=n), out=ptr[1:])
    return ptr.astype(np.int32), c.astype(np.int32)


@pytest.mark.parametrize("symmetric", [False, True])
def test_tier_lists_many_chunks(sporder, symmetric):
    """More chunks than one classification workgroup orders (8192): the tier-2
    and global-path lists are built by a grid of workgroups, and chunks of all
    three tiers (hub rows of 7000 to 12000 nonzeros in chunks of 4 rows) are
    sketched concurrently.  Bit-exact table and permutation."""
    hubs = {5: 12000, 6: 9000, 20000: 12000, 20001: 12000, 20002: 10000, 39998: 7000}
    ptr, ind = hub_matrix(40000, 8, hubs, 41, symmetric)
    assert synth.is_pattern_symmetric(ptr, ind) == symmetric
    chunk = 4
    E = ptr[np.minimum(np.arange(0, 40000, chunk) + chunk, 40000)] - ptr[np.arange(0, 40000, chunk)]
    assert E.size > 8192 and (E > 16384).any() and (E > 32768).any()
    check_table(sporder, ptr, ind, 16, 4.0, chunk, symmetric)
    dptr, dind = dev_csr(ptr, ind)
    g = sporder.chunk_similarity_greedy(dptr, dind, is_symmetric=symmetric, k=16,
                                        oversampling=4.0, chunk_size=chunk)
    o, _ = oracle.chunk_similarity_greedy(ptr, ind, is_symmetric=symmetric, k=16,
                                          oversampling=4.0, chunk_size=chunk)
    assert np.array_equal(g.cpu().numpy(), o)


def test_greedy_compact_overflow_entries(sporder):
    """A chunk whose top-k slice has more valid entries than the compact LDS
    capacity (8192 entries when there are few chunks) reads entries from
    global memory: same order."""
    ptr, ind = dense_random(4096, 12, 32, True)
    for chunk in (4096, 4000):
        dptr, dind = dev_csr(ptr, ind)
        g, s = sporder.chunk_similarity_greedy(dptr, dind, is_symmetric=True, chunk_size=chunk,
                                               with_stats=True)
        o, os_ = oracle.chunk_similarity_greedy(ptr, ind, is_symmetric=True, chunk_size=chunk)
        assert s["avg_degree"] * 4096 > 8192
        assert np.array_equal(g.cpu().numpy(), o)


def block_random(n, block, deg, seed):
    """Symmetric pattern whose columns stay inside diagonal blocks of `block`
    rows, so a row's table entries are rows of its own block."""
    rng = np.random.default_rng(seed)
    rows = np.repeat(np.arange(n), deg)
    cols = (rows // block) * block + rng.integers(0, block, size=n * deg)
    cols = np.minimum(cols, n - 1)
    rows, cols = np.concatenate([rows, cols]), np.concatenate([cols, rows])
    keys = np.unique(rows.astype(np.int64) * n + cols)
    r, c = keys // n, keys % n
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(np.bincount(r, minlength=n), out=ptr[1:])
    return ptr.astype(np.int32), c.astype(np.int32)


def in_chunk_totals(ptr, ind, k, chunk):
    n = ptr.shape[0] - 1
    idx, _ = oracle.unpack_table(oracle.chunk_similarity_top_k(ptr, ind, k, chunk, 4.0, True))
    inside = (idx >= 0) & (idx // chunk == np.arange(n)[:, None] // chunk)
    return np.add.reduceat(inside.sum(1), np.arange(0, n, chunk))


@pytest.mark.parametrize("case", ["few_chunks", "many_chunks"])
def test_greedy_staging_capacity(sporder, case):
    """Slices of 2049 to 8192 in-chunk entries: with at most two chunks per CU
    the chain stages up to 8192 entries in LDS; with more chunks it stages
    2048 64-bit entries, and past that walks a packed slice (16-bit local
    indices in preference order, runs of equal weight sorted by index) when
    no statistics are asked for, or reads the rows from global memory when
    they are.  Same order every way, and the same restart count."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if case == "few_chunks":
        chunk, n, block = 1024, 8 * 1024, 6
    else:
        chunk, n, block = 256, 256 * (2 * cus + 64), 24
    print(f"[staging] {case} n={n} chunk={chunk} block={block} cus={cus}", flush=True)
    ptr, ind = block_random(n, block, 4, 51)
    tot = in_chunk_totals(ptr, ind, 16, chunk)
    assert tot.min() > 2048 and tot.max() <= 8192
    dptr, dind = dev_csr(ptr, ind)
    o, os_ = oracle.chunk_similarity_greedy(ptr, ind, is_symmetric=True, k=16, oversampling=4.0,
                                            chunk_size=chunk)
    g = sporder.chunk_similarity_greedy(dptr, dind, is_symmetric=True, k=16, oversampling=4.0,
                                        chunk_size=chunk)
    assert np.array_equal(g.cpu().numpy(), o)
    g2, s = sporder.chunk_similarity_greedy(dptr, dind, is_symmetric=True, k=16,
                                            oversampling=4.0, chunk_size=chunk, with_stats=True)
    assert np.array_equal(g2.cpu().numpy(), o)
    assert s["chain_restarts"] == os_["chain_restarts"]


def block_parts(n, seed, specs):
    """Equal row ranges of block-local random patterns, (block, degree) each,
    stacked on the diagonal: slices of very different density in one matrix."""
    sizes = [n // len(specs)] * len(specs)
    sizes[-1] = n - sum(sizes[:-1])
    ptr, inds, nnz, off = [np.zeros(1, np.int64)], [], 0, 0
    for (block, deg), h in zip(specs, sizes):
        p, i = block_random(h, block, deg, seed)
        seed += 1
        ptr.append(p[1:].astype(np.int64) + nnz)
        inds.append(i.astype(np.int64) + off)
        nnz += int(p[-1])
        off += h
    return np.concatenate(ptr).astype(np.int32), np.concatenate(inds).astype(np.int32)


def test_greedy_split_launches(sporder):
    """One call whose 1024-row slices hold S valid entries in every range the
    chain tells apart (k 24): S <= 2048 (64-bit staging), 2048 < S <= 8192
    (packed within the first launch's LDS), 8192 < S <= 16384 (the second,
    packed launch) and S > 16384 (rows read from the table).  Each launch takes
    exactly its own chunks and skips the other's."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    chunk, k = 1024, 24
    n = chunk * (2 * cus + 40)
    ptr, ind = block_parts(n, 60, [(64, 12), (16, 3), (12, 2), (4, 1)])
    tot = in_chunk_totals(ptr, ind, k, chunk)
    print(f"[split] n={n} slices {tot.min()}..{tot.max()}", flush=True)
    for lo, hi in ((0, 2048), (2048, 8192), (8192, 16384), (16384, 1 << 30)):
        assert ((tot > lo) & (tot <= hi)).sum() > 50, (lo, hi)
    dptr, dind = dev_csr(ptr, ind)
    g = sporder.chunk_similarity_greedy(dptr, dind, is_symmetric=True, k=k, oversampling=4.0,
                                        chunk_size=chunk)
    o, _ = oracle.chunk_similarity_greedy(ptr, ind, is_symmetric=True, k=k, oversampling=4.0,
                                          chunk_size=chunk)
    assert np.array_equal(g.cpu().numpy(), o)


@pytest.mark.parametrize("k", [16, 32])
def test_greedy_packed_slices(sporder, k):
    """Many chunks whose slices pass the 2048-entry staging capacity, on
    patterns with many equal weights (block-local random rows: rows of one
    block share columns, and degrees repeat): the packed walk (no
    statistics) must order each run of equal weight by local index.  Also
    sporder-cg, whose global table mixes out-of-chunk entries into the rows
    (filtered when the slice is packed).  Bit-exact against the oracle."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    chunk = 256
    n = chunk * (2 * cus + 40)
    ptr, ind = block_random(n, 32, 5, 52)
    tot = in_chunk_totals(ptr, ind, k, chunk)
    print(f"[packed] n={n} k={k} in-chunk entries per slice {tot.min()}..{tot.max()}", flush=True)
    assert tot.min() > 2048
    dptr, dind = dev_csr(ptr, ind)
    g = sporder.chunk_similarity_greedy(dptr, dind, is_symmetric=True, k=k, oversampling=2.0,
                                        chunk_size=chunk)
    o, _ = oracle.chunk_similarity_greedy(ptr, ind, is_symmetric=True, k=k, oversampling=2.0,
                                          chunk_size=chunk)
    assert np.array_equal(g.cpu().numpy(), o)
    g = sporder.chunk_greedy(dptr, dind, is_symmetric=True, k=k, oversampling=2.0,
                             chunk_size=chunk)
    o, _ = oracle.chunk_greedy(ptr, ind, is_symmetric=True, k=k, oversampling=2.0,
                               chunk_size=chunk)
    assert np.array_equal(g.cpu().numpy(), o)


def drop_one_mirror(ptr, ind, chunk):
    """Remove one nonzero (a, b), a < b in one chunk, whose mirror (b, a) stays."""
    n = ptr.shape[0] - 1
    rows = np.repeat(np.arange(n), np.diff(ptr))
    pick = np.nonzero((ind > rows) & (ind // chunk == rows // chunk))[0][0]
    keep = np.ones(ind.shape[0], bool)
    keep[pick] = False
    p = ptr.astype(np.int64).copy()
    p[rows[pick] + 1:] -= 1
    return p.astype(np.int32), ind[keep]


def asymmetric_cases():
    """Non-symmetric patterns passed with is_symmetric=True: (ptr, ind, chunk)."""
    hubs = {5: 12000, 6: 9000, 20000: 12000, 20001: 12000, 20002: 10000, 39998: 7000}
    st = synth.stencil7(20, 13, scramble=False)[:2]
    return {
        "one_missing_mirror_local": (*drop_one_mirror(*st, 256), 256),
        "random_local_and_overflow_4096": (*dense_random(12000, 40, 31, False), 4096),
        "random_local_and_overflow_1500": (*dense_random(12000, 40, 31, False), 1500),
        "hubs_three_tiers": (*hub_matrix(40000, 8, hubs, 41, False), 4),
    }


ASYM = asymmetric_cases()


@pytest.mark.parametrize("name", sorted(ASYM))
def test_is_symmetric_on_asymmetric_pattern_reads_csr_as_csc(sporder, name):
    """is_symmetric=True on a pattern that is not symmetric: the reference
    reads the CSR as its own CSC for every chunk (csr2csc.h:49-59).  The
    chunk-local tiers would build the true transpose, so the mirror check
    sends such a call through the global path; table, csg order and stats
    equal the oracle's CSR-as-CSC result.  Each case is one the true
    transpose would change (checked on the oracle)."""
    ptr, ind, chunk = ASYM[name]
    assert not synth.is_pattern_symmetric(ptr, ind)
    k, ovs = 16, 4.0
    as_csc = oracle.chunk_similarity_top_k(ptr, ind, k, chunk, ovs, is_symmetric=True)
    transposed = oracle.chunk_similarity_top_k(ptr, ind, k, chunk, ovs, is_symmetric=False)
    assert not np.array_equal(as_csc, transposed)
    check_table(sporder, ptr, ind, k, ovs, chunk, True)
    dptr, dind = dev_csr(ptr, ind)
    g, s = sporder.chunk_similarity_greedy(dptr, dind, is_symmetric=True, k=k, oversampling=ovs,
                                           chunk_size=chunk, with_stats=True)
    o, os_ = oracle.chunk_similarity_greedy(ptr, ind, is_symmetric=True, k=k, oversampling=ovs,
                                            chunk_size=chunk)
    assert np.array_equal(g.cpu().numpy(), o)
    assert s["chain_restarts"] == os_["chain_restarts"]
    assert s["zero_degree_rows"] == os_["zero_degree_rows"]
    g2 = sporder.chunk_greedy(dptr, dind, is_symmetric=True, k=k, oversampling=ovs,
                              chunk_size=chunk)
    o2, _ = oracle.chunk_greedy(ptr, ind, is_symmetric=True, k=k, oversampling=ovs,
                                chunk_size=chunk)
    assert np.array_equal(g2.cpu().numpy(), o2)


def test_is_symmetric_one_chunk_similarity_graph(sporder):
    """The one-chunk global sketch (similarity_graph, n within the LDS tiers)
    with is_symmetric=True on a non-symmetric pattern equals the oracle's
    CSR-as-CSC table; the same call on the symmetric pattern stays on the
    chunk-local tier and is still exact."""
    ptr, ind = dense_random(3000, 6, 71, False)
    sptr, sind = dense_random(3000, 3, 71, True)
    for p, i in ((ptr, ind), (sptr, sind)):
        n = p.shape[0] - 1
        dptr, dind = dev_csr(p, i)
        gi, gw = sporder.similarity_graph(dptr, dind, is_symmetric=True, k=16, oversampling=2.0)
        oi, ow = oracle.unpack_table(
            oracle.chunk_similarity_top_k(p, i, 16, n, 2.0, is_symmetric=True))
        assert np.array_equal(gi.cpu().numpy(), oi)
        assert np.array_equal(weight_bits(gw.cpu().numpy()), weight_bits(ow))


def distinct_candidates_matrix(n, D):
    """Row 0 holds columns n-1, n-2, n-3; row j in 1..D holds n-1, plus n-2
    when j is odd and n-3 when j is a multiple of 3.  Row 0's stream is then
    the D rows in ascending order, the odd rows, the multiples of 3: exactly D
    distinct candidates with one, two or three occurrences and three Dice
    weights (rows of one, two or three nonzeros).  The other rows are empty."""
    rows, cols = [0, 0, 0], [n - 1, n - 2, n - 3]
    for j in range(1, D + 1):
        rows.append(j)
        cols.append(n - 1)
        if j % 2:
            rows.append(j)
            cols.append(n - 2)
        if j % 3 == 0:
            rows.append(j)
            cols.append(n - 3)
    rows, cols = np.array(rows), np.array(cols)
    order = np.lexsort((cols, rows))
    rows, cols = rows[order], cols[order]
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(np.bincount(rows, minlength=n), out=ptr[1:])
    return ptr.astype(np.int32), cols.astype(np.int32)


@pytest.mark.parametrize("k,ovs", [(16, 4.0), (24, 4.0), (32, 4.0)])
@pytest.mark.parametrize("extra", [-1, 0, 1, 2])
@pytest.mark.parametrize("chunk", [1024, 5000])
def test_sketch_capacity_boundary(sporder, k, ovs, extra, chunk):
    """Rows with M - 1, M, M + 1 and M + 2 distinct candidates (M = the
    sketch capacity: 64, 96, 128): no eviction up to M, then the first
    evictions, whose victim is the smallest weight with ties to the lowest
    (cell, lane), and whose newcomer inherits its weight.  Chunks of 1024
    rows take the chunk-local tier, chunks of 5000 the global path.  Tables
    bit-exact against the oracle; row 0's distinct count checked on the
    host."""
    M = ((int(k * ovs) + 31) // 32) * 32
    D = M + extra
    n = 5000
    ptr, ind = distinct_candidates_matrix(n, D)
    # Row 0's stream on the host: the rows of each of its columns, minus itself.
    stream = [r for c in ind[ptr[0]:ptr[1]]
              for r in range(n) if r != 0 and c in ind[ptr[r]:ptr[r + 1]]]
    assert len(set(stream)) == D and len(stream) == D + (D + 1) // 2 + D // 3
    oi, ow = check_table(sporder, ptr, ind, k, ovs, chunk, False)
    # Row 0 keeps its k heaviest candidates; the rows seen three times lead.
    assert (oi[0] >= 0).sum() == k
    assert set(oi[0, :3].tolist()) <= {j for j in range(1, D + 1) if j % 6 == 3}
