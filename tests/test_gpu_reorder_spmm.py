"""GPU parity of the permutation apply and the CSR SpMM.

Reorder: bit-exact against the oracle (integers and copied fp32 values).
SpMM row-split: bit-exact against the oracle's stated order (fmaf chains in
CSR order, rows past SPORDER_SPMM_LONG_ROW in segments added left to right); both
variants within 1e-5 relative of an fp64 reference (the tolerance north_star
states for fp32 SpMM).
"""

import time

import numpy as np
import pytest
import torch

import oracle
from chunkedgreedy_amd import synth

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def long_row_matrix(n=20000, seed=7):
    """Rows of 0, 1, 63, 64, 65, 300, 4096, 4097 and 12000 entries."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(0, 20, size=n)
    for i, L in enumerate([0, 1, 63, 64, 65, 300, 4096, 4097, 12000]):
        lens[i * 37] = L
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(lens, out=ptr[1:])
    ind = np.concatenate([np.sort(rng.choice(n, size=L, replace=False)) for L in lens])
    val = rng.standard_normal(ind.shape[0]).astype(np.float32)
    return ptr.astype(np.int32), ind.astype(np.int32), val


def hub_matrix(n=300_000, hub=250_000, seed=8):
    """Row 0 holds `hub` entries (489 SpMM segments), the rest 0..8 each."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(0, 9, size=n)
    lens[0] = hub
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(lens, out=ptr[1:])
    ind = np.concatenate([np.sort(rng.choice(n, size=L, replace=False)) for L in lens])
    val = rng.standard_normal(ind.shape[0]).astype(np.float32)
    return ptr.astype(np.int32), ind.astype(np.int32), val


def many_huge_matrix(n=60000, seed=9):
    """40 rows of 4097..9000 entries (all sorted together past the LDS sort)
    among rows of 0..10."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(0, 11, size=n)
    lens[rng.choice(n, size=40, replace=False)] = rng.integers(4097, 9001, size=40)
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(lens, out=ptr[1:])
    ind = np.concatenate([np.sort(rng.choice(n, size=L, replace=False)) for L in lens])
    val = rng.standard_normal(ind.shape[0]).astype(np.float32)
    return ptr.astype(np.int32), ind.astype(np.int32), val


def skewed_matrix(n=50000, seed=10):
    """80 % of rows with 0..4 entries, 20 % with 60..120: a mean past 16, so
    rows of at most 4 entries take the one-lane pass of the permutation."""
    rng = np.random.default_rng(seed)
    lens = np.where(rng.random(n) < 0.8, rng.integers(0, 5, size=n),
                    rng.integers(60, 121, size=n))
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(lens, out=ptr[1:])
    assert ptr[-1] / n >= 17
    ind = np.concatenate([np.sort(rng.choice(n, size=L, replace=False)) for L in lens])
    val = rng.standard_normal(ind.shape[0]).astype(np.float32)
    return ptr.astype(np.int32), ind.astype(np.int32), val


def mats():
    return {
        "skewed": skewed_matrix(),
        "C1": synth.config1(21),
        "rmat12": synth.rmat(12, 16, 22),
        "stencil16": synth.stencil7(16, 23),
        "longrows": long_row_matrix(),
        "hub": hub_matrix(),
        "manyhuge": many_huge_matrix(),
    }


MATS = mats()


def permutation(n, kind, seed=5):
    """A uniform permutation, or one that shuffles rows only inside windows:
    aligned windows of 1024 (as csg's chains do inside their chunks) or 8192
    keep every column inside an aligned block of 2^10 or 2^13 indices (the
    apply's run mode); aligned windows of 16384 move indices by less than
    2^15 (16-bit column remap) but past run mode's largest block; windows of
    1000 are not aligned to a power of two (the blocks they stay inside
    depend on where a window crosses one); "identity" moves nothing."""
    rng = np.random.default_rng(seed)
    if kind == "uniform":
        return rng.permutation(n).astype(np.int32)
    if kind == "identity":
        return np.arange(n, dtype=np.int32)
    width = {"windowed": 1024, "windowed8192": 8192, "windowed16384": 16384,
             "unaligned1000": 1000}[kind]
    perm = np.arange(n)
    for w in range(0, n, width):
        rng.shuffle(perm[w:w + width])
    return perm.astype(np.int32)


def _reorder_check(sporder, ptr, ind, val, perm, symmetric, with_val):
    if with_val:
        gp, gi, gv = sporder.reorder(t(ptr), t(ind), t(perm), val=t(val), symmetric=symmetric)
        op, oi, ov = oracle.reorder(ptr, ind, perm, val=val, symmetric=symmetric)
        assert np.array_equal(gv.cpu().numpy().view(np.uint32), ov.view(np.uint32))
    else:
        gp, gi = sporder.reorder(t(ptr), t(ind), t(perm), symmetric=symmetric)
        op, oi = oracle.reorder(ptr, ind, perm, symmetric=symmetric)
    assert np.array_equal(gp.cpu().numpy(), op)
    assert np.array_equal(gi.cpu().numpy(), oi)


@pytest.mark.parametrize("name", sorted(MATS))
@pytest.mark.parametrize("symmetric", [False, True])
@pytest.mark.parametrize("with_val", [False, True])
@pytest.mark.parametrize("kind", ["uniform", "windowed"])
def test_reorder_bit_exact(sporder, name, symmetric, with_val, kind):
    """Every size class of row (register, wave, workgroup and device-wide
    sorts; big-row copies), both column remaps (32-bit when some index moves
    by 2^15 or more, 16-bit deltas otherwise), with and without values."""
    ptr, ind, val = MATS[name]
    n = ptr.shape[0] - 1
    perm = permutation(n, kind)
    print(f"[reorder] {name} sym={symmetric} val={with_val} perm={kind}", flush=True)
    if with_val:
        gp, gi, gv = sporder.reorder(t(ptr), t(ind), t(perm), val=t(val), symmetric=symmetric)
        op, oi, ov = oracle.reorder(ptr, ind, perm, val=val, symmetric=symmetric)
        assert np.array_equal(gv.cpu().numpy().view(np.uint32), ov.view(np.uint32))
    else:
        gp, gi = sporder.reorder(t(ptr), t(ind), t(perm), symmetric=symmetric)
        op, oi = oracle.reorder(ptr, ind, perm, symmetric=symmetric)
    assert np.array_equal(gp.cpu().numpy(), op)
    assert np.array_equal(gi.cpu().numpy(), oi)


@pytest.mark.parametrize("name", ["longrows", "hub", "manyhuge", "rmat12", "skewed"])
@pytest.mark.parametrize("kind", ["identity", "windowed8192", "windowed16384", "unaligned1000",
                                  "csg", "cg"])
def test_reorder_block_runs(sporder, name, kind):
    """SYMMETRIC with values under permutations that keep columns inside
    aligned blocks (run mode: rows of 2G+1..512, 513..4096 and past 4096
    entries, singleton runs, runs placed by counting, by the wave sort and
    by the LDS bitmap) and ones that do not (full sorts): csg's and cg's own
    orders of the matrix, the identity, and windowed shuffles."""
    ptr, ind, val = MATS[name]
    n = ptr.shape[0] - 1
    if kind in ("csg", "cg"):
        fn = sporder.chunk_similarity_greedy if kind == "csg" else sporder.chunk_greedy
        perm = fn(t(ptr), t(ind)).cpu().numpy().astype(np.int32)
    else:
        perm = permutation(n, kind)
    print(f"[reorder runs] {name} perm={kind}", flush=True)
    _reorder_check(sporder, ptr, ind, val, perm, True, True)


def unsorted_rows_matrix(n=30000, seed=11):
    """Distinct columns, but rows 5 (300 entries), 40 (5000 entries, the
    device-wide class) and 90 (2000 entries) not in increasing order: one
    pair swapped, the whole row reversed, a run's order rotated."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(0, 12, size=n)
    lens[5], lens[40], lens[90] = 300, 5000, 2000
    rows = [np.sort(rng.choice(n, size=L, replace=False)) for L in lens]
    rows[5][[100, 101]] = rows[5][[101, 100]]
    rows[40] = rows[40][::-1].copy()
    rows[90] = np.concatenate([rows[90][1:], rows[90][:1]])
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(lens, out=ptr[1:])
    ind = np.concatenate(rows)
    val = rng.standard_normal(ind.shape[0]).astype(np.float32)
    return ptr.astype(np.int32), ind.astype(np.int32), val


@pytest.mark.parametrize("kind", ["windowed", "identity", "uniform"])
def test_reorder_unsorted_input_rows(sporder, kind):
    """Input rows that are not strictly increasing: run mode detects them and
    the call takes the full sorts; the output is sorted like the oracle's."""
    ptr, ind, val = unsorted_rows_matrix()
    perm = permutation(ptr.shape[0] - 1, kind)
    print(f"[reorder unsorted] perm={kind}", flush=True)
    _reorder_check(sporder, ptr, ind, val, perm, True, True)


def test_reorder_csg_roundtrip(sporder):
    """csg order -> P A P^T -> inverse permutation restores A exactly."""
    ptr, ind, val = MATS["C1"]
    order = sporder.chunk_similarity_greedy(t(ptr), t(ind))
    p1, i1, v1 = sporder.reorder(t(ptr), t(ind), order, val=t(val), symmetric=True)
    inv = torch.empty_like(order)
    inv[order.long()] = torch.arange(order.numel(), dtype=torch.int32, device=DEV)
    p2, i2, v2 = sporder.reorder(p1, i1, inv, val=v1, symmetric=True)
    assert torch.equal(p2.cpu(), t(ptr).cpu())
    assert torch.equal(i2.cpu(), t(ind).cpu())
    assert torch.equal(v2.cpu(), t(val).cpu())


def test_reorder_rejects_bad_lengths(sporder):
    ptr, ind, _ = MATS["C1"]
    with pytest.raises(ValueError):
        sporder.reorder(t(ptr), t(ind), t(np.arange(10, dtype=np.int32)))


@pytest.mark.parametrize("name", sorted(MATS))
@pytest.mark.parametrize("N", [1, 3, 4, 8, 16, 32, 64, 128, 256, 260])
def test_spmm_rowsplit_bit_exact(sporder, name, N):
    ptr, ind, val = MATS[name]
    n = ptr.shape[0] - 1
    B = np.random.default_rng(N).standard_normal((n, N)).astype(np.float32)
    print(f"[spmm] {name} N={N}", flush=True)
    C, ms = sporder.spmm_csr(t(ptr), t(ind), t(val), t(B), algo="row_split")
    ref = oracle.spmm_csr(ptr, ind, val, B)
    assert np.array_equal(C.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    assert ms > 0.0


@pytest.mark.parametrize("name", sorted(MATS))
@pytest.mark.parametrize("N", [3, 8, 32, 128, 260])
@pytest.mark.parametrize("sides", ["both", "row", "col"])
def test_spmm_scaled_equals_unfused(sporder, name, N, sides):
    """diag(rs) A diag(cs) B in one call equals, bit for bit, the three steps
    it replaces (cs * B elementwise, the row-split SpMM, rs * C elementwise),
    both on the GPU and from the oracle with numpy's fp32 products; every
    kernel of the row-split is reached (the scalar path at N = 3, the dynamic
    claim at N <= 32, the fixed row groups at 128 and in two column passes at
    260, the long-row segments and fixup)."""
    ptr, ind, val = MATS[name]
    n = ptr.shape[0] - 1
    rng = np.random.default_rng(100 + N)
    B = rng.standard_normal((n, N)).astype(np.float32)
    rs = rng.uniform(0.05, 2.0, n).astype(np.float32) if sides in ("both", "row") else None
    cs = rng.uniform(0.05, 2.0, n).astype(np.float32) if sides in ("both", "col") else None
    print(f"[spmm_scaled] {name} N={N} {sides}", flush=True)
    C, ms = sporder.spmm_csr_scaled(t(ptr), t(ind), t(val), t(B),
                                    row_scale=None if rs is None else t(rs),
                                    col_scale=None if cs is None else t(cs))
    Bp = t(B) if cs is None else (t(cs)[:, None] * t(B)).contiguous()
    C1, _ = sporder.spmm_csr(t(ptr), t(ind), t(val), Bp, algo="row_split")
    want = C1 if rs is None else t(rs)[:, None] * C1
    got = C.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.cpu().numpy().view(np.uint32))
    Bn = B if cs is None else cs[:, None] * B
    ref = oracle.spmm_csr(ptr, ind, val, Bn)
    ref = ref if rs is None else rs[:, None] * ref
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert ms > 0.0
    if cs is not None:
        # The per-nonzero form the kernels read, given directly.
        C2, _ = sporder.spmm_csr_scaled(t(ptr), t(ind), t(val), t(B),
                                        row_scale=None if rs is None else t(rs),
                                        nz_col_scale=t(cs[ind]))
        assert torch.equal(C2.view(torch.int32), C.view(torch.int32))


def test_spmm_scaled_rejects_bad_scales(sporder):
    ptr, ind, val = MATS[sorted(MATS)[0]]
    n = ptr.shape[0] - 1
    B = t(np.ones((n, 4), np.float32))
    with pytest.raises(ValueError):
        sporder.spmm_csr_scaled(t(ptr), t(ind), t(val), B, row_scale=t(np.ones(n - 1, np.float32)))
    with pytest.raises(ValueError):
        sporder.spmm_csr_scaled(t(ptr), t(ind), t(val), B,
                                col_scale=torch.ones(n, dtype=torch.float64, device=DEV))
    with pytest.raises(ValueError):
        sporder.spmm_csr_scaled(t(ptr), t(ind), t(val), B,
                                nz_col_scale=t(np.ones(n, np.float32)))  # n, not nnz
    with pytest.raises(ValueError):
        sporder.spmm_csr_scaled(t(ptr), t(ind), t(val), B, col_scale=t(np.ones(n, np.float32)),
                                nz_col_scale=t(np.ones(ind.shape[0], np.float32)))


def rel_err(c, ref64):
    scale = np.abs(ref64).max() + 1e-30
    return np.abs(c.astype(np.float64) - ref64).max() / scale


@pytest.mark.parametrize("name", sorted(MATS))
@pytest.mark.parametrize("N", [4, 32, 128, 33])
def test_spmm_merge_path_tolerance(sporder, name, N):
    ptr, ind, val = MATS[name]
    n = ptr.shape[0] - 1
    import scipy.sparse as sps

    B = np.random.default_rng(N + 1).standard_normal((n, N)).astype(np.float32)
    A = sps.csr_matrix((val.astype(np.float64), ind, ptr), shape=(n, n))
    ref64 = A @ B.astype(np.float64)
    C, _ = sporder.spmm_csr(t(ptr), t(ind), t(val), t(B), algo="merge_path")
    assert rel_err(C.cpu().numpy(), ref64) < 1e-5
    C2, _ = sporder.spmm_csr(t(ptr), t(ind), t(val), t(B), algo="row_split")
    assert rel_err(C2.cpu().numpy(), ref64) < 1e-5


def test_bench_hook(sporder):
    """The hook's mean time per repeat: positive, the inputs untouched, growing
    with the width (N = 256 against N = 16 on a 2^18-row matrix), and within a
    factor of four of the same SpMM timed from outside."""
    ptr, ind, _ = MATS["C1"]
    dptr, dind = t(ptr), t(ind)
    ms = sporder.bench_cusparse_spmm(dptr, dind, 32, warmup=1, repeat=3, seed=7)
    assert ms > 0.0
    assert np.array_equal(dptr.cpu().numpy(), ptr) and np.array_equal(dind.cpu().numpy(), ind)
    with pytest.raises(ValueError):
        sporder.bench_cusparse_spmm(dptr, dind, 0)
    p2, i2, v2 = synth.planted(1 << 18, 4096, 16, 31)
    dp, di = t(p2), t(i2)
    narrow = sporder.bench_cusparse_spmm(dp, di, 16, warmup=3, repeat=20, seed=1)
    wide = sporder.bench_cusparse_spmm(dp, di, 256, warmup=3, repeat=20, seed=1)
    assert wide > narrow > 0.0
    B = torch.rand((p2.shape[0] - 1, 256), device=DEV)
    out = torch.empty_like(B)
    dv = t(v2)
    for _ in range(3):
        sporder.spmm_csr(dp, di, dv, B, out=out)
    # Each call ends in a synchronize of the library stream: host wall time.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(20):
        sporder.spmm_csr(dp, di, dv, B, out=out)
    torch.cuda.synchronize()
    outside = (time.perf_counter() - t0) * 1e3 / 20
    assert 0.25 < wide / outside < 4.0, (wide, outside)


def test_reorder_row_offsets_past_direct_scan(sporder):
    """More than 4096 scan tiles of 4096 offsets (n = 2^24 + 5000 rows of 0..2
    entries): the offset scan takes its three-pass form, where each tile's
    offset comes from one workgroup's scan of the tile totals.  Offsets equal
    NumPy's cumulative sum, entries the gathered rows."""
    n = (1 << 24) + 5000
    rng = np.random.default_rng(12)
    lens = rng.integers(0, 3, size=n).astype(np.int64)
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(lens, out=ptr[1:])
    ind = rng.integers(0, n, size=int(ptr[-1])).astype(np.int32)
    perm = rng.permutation(n).astype(np.int32)
    gp, gi = sporder.reorder(t(ptr.astype(np.int32)), t(ind), t(perm))
    want_ptr = np.zeros(n + 1, np.int64)
    np.cumsum(lens[perm], out=want_ptr[1:])
    assert np.array_equal(gp.cpu().numpy(), want_ptr.astype(np.int32))
    starts = ptr[perm]
    rows = np.repeat(np.arange(n), lens[perm])
    want_ind = ind[starts[rows] + (np.arange(rows.size) - want_ptr[rows])]
    assert np.array_equal(gi.cpu().numpy(), want_ind)
