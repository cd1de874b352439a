"""The oracle's transpose, permutation apply and SpMM against scipy / fp64."""

import numpy as np
import pytest
import scipy.sparse as sp

import oracle
from chunkedgreedy_amd import synth


def scipy_csr(ptr, ind, val):
    n = ptr.shape[0] - 1
    return sp.csr_matrix((val, ind, ptr), shape=(n, n))


MATS = {
    "C1": synth.config1(5),
    "rmat10": synth.rmat(10, 16, 6),
    "stencil6": synth.stencil7(6, 7),
    "empty_rows": (np.array([0, 0, 2, 2, 5], np.int32), np.array([1, 3, 0, 1, 3], np.int32),
                   np.array([1, 2, 3, 4, 5], np.float32)),
}


@pytest.mark.parametrize("name", sorted(MATS))
def test_csr2csc_matches_scipy(name):
    ptr, ind, val = MATS[name]
    cptr, rind = oracle.csr2csc(ptr, ind)
    t = scipy_csr(ptr, ind, val).tocsc()
    t.sort_indices()
    assert np.array_equal(cptr, t.indptr) and np.array_equal(rind, t.indices)


@pytest.mark.parametrize("name", sorted(MATS))
@pytest.mark.parametrize("symmetric", [False, True])
def test_reorder_matches_scipy(name, symmetric):
    ptr, ind, val = MATS[name]
    n = ptr.shape[0] - 1
    perm = np.random.default_rng(1).permutation(n).astype(np.int32)
    p2, i2, v2 = oracle.reorder(ptr, ind, perm, val=val, symmetric=symmetric)
    a = scipy_csr(ptr, ind, val)
    ref = a[perm, :][:, perm] if symmetric else a[perm, :]
    ref = ref.tocsr()
    ref.sort_indices()
    assert np.array_equal(p2, ref.indptr)
    assert np.array_equal(i2, ref.indices)
    assert np.array_equal(v2, ref.data.astype(np.float32))


def test_reorder_without_values_and_zero_fill():
    ptr, ind, val = MATS["C1"]
    n = ptr.shape[0] - 1
    perm = np.arange(n, dtype=np.int32)[::-1].copy()
    p2, i2 = oracle.reorder(ptr, ind, perm)
    p3, i3, _ = oracle.reorder(ptr, ind, perm, val=val)
    assert np.array_equal(p2, p3) and np.array_equal(i2, i3)


@pytest.mark.parametrize("name", sorted(MATS))
@pytest.mark.parametrize("N", [1, 5, 32])
def test_spmm_matches_fp64(name, N):
    ptr, ind, val = MATS[name]
    n = ptr.shape[0] - 1
    B = np.random.default_rng(N).standard_normal((n, N)).astype(np.float32)
    C = oracle.spmm_csr(ptr, ind, val, B)
    ref = scipy_csr(ptr, ind, val.astype(np.float64)) @ B.astype(np.float64)
    scale = np.abs(ref).max() + 1e-30
    assert np.abs(C - ref).max() / scale < 1e-5


def round_f32(x):
    """Correctly rounded (nearest, ties to even) fp32 value of a Fraction."""
    from fractions import Fraction

    f = np.float32(float(x))
    best = None
    for c in (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))):
        d = abs(Fraction(float(c)) - x)
        key = (d, int(c.view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return best[1]


def stated_order_row(ptr, ind, val, B, r, j, long_row=512, seg_len=512):
    """Row r, column j of A @ B in the stated order, with every fmaf and every
    partial add done in exact rational arithmetic and rounded once to fp32."""
    from fractions import Fraction

    s, e = int(ptr[r]), int(ptr[r + 1])
    seg = seg_len if e - s > long_row else max(e - s, 1)
    total = None
    q0 = s
    while q0 < e or q0 == s:
        acc = np.float32(0.0)
        for p in range(q0, min(q0 + seg, e)):
            exact = Fraction(float(val[p])) * Fraction(float(B[ind[p], j])) + Fraction(float(acc))
            acc = round_f32(exact)
        total = acc if total is None else round_f32(Fraction(float(total)) + Fraction(float(acc)))
        q0 += seg
    return total


def test_spmm_fmaf_order():
    """Each output of a short row is a left-to-right fmaf chain in CSR order:
    check the longest row against exact arithmetic rounded once per step."""
    ptr, ind, val = MATS["rmat10"]
    n = ptr.shape[0] - 1
    assert np.diff(ptr).max() <= 512
    B = np.random.default_rng(9).standard_normal((n, 3)).astype(np.float32)
    C = oracle.spmm_csr(ptr, ind, val, B)
    r = int(np.argmax(np.diff(ptr)))
    for j in range(3):
        acc = stated_order_row(ptr, ind, val, B, r, j)
        assert C[r, j].view(np.uint32) == acc.view(np.uint32)


def long_rows_matrix(lengths, n, seed):
    rng = np.random.default_rng(seed)
    ptr = np.zeros(len(lengths) + 1, np.int64)
    np.cumsum(lengths, out=ptr[1:])
    ind = np.concatenate([np.sort(rng.choice(n, size=d, replace=False)) for d in lengths])
    val = rng.uniform(-1, 1, ind.shape[0]).astype(np.float32)
    return ptr.astype(np.int32), ind.astype(np.int32), val


def test_spmm_long_rows_stated_order():
    """Rows around and past the long-row threshold (511 .. 1537 nonzeros)
    against the stated order in exact arithmetic: segments of 512 from the row
    start, chains added left to right.  A segment length off by one, a
    different threshold or a different order of the partial sums changes the
    rounding of these random rows."""
    lengths = [511, 512, 513, 1024, 1100, 1537]
    n = 2000
    ptr, ind, val = long_rows_matrix(lengths, n, 3)
    # Pad to a square matrix: rows beyond len(lengths) are empty.
    ptr = np.concatenate([ptr, np.full(n - len(lengths), ptr[-1], np.int32)])
    B = np.random.default_rng(4).standard_normal((n, 2)).astype(np.float32)
    C = oracle.spmm_csr(ptr, ind, val, B)
    for r in range(len(lengths)):
        for j in range(2):
            want = stated_order_row(ptr, ind, val, B, r, j)
            assert C[r, j].view(np.uint32) == want.view(np.uint32), (lengths[r], j)
    assert not C[len(lengths):].any()


def test_spmm_segment_boundary_known_answer():
    """A row of 1024 ones against B = [1, 2^-25 x 1023]: one chain rounds every
    tiny term away (1.0); segments of 512 give 1 + 511*2^-25 -> 1.0 for the
    first and exactly 2^-16 for the second, so the row is 1 + 2^-16.  With 256
    the row would be 1 + 3*2^-17; a row of 512 stays one chain (1.0)."""
    n = 1024
    for d, want in ((1024, np.float32(1.0) + np.float32(2.0 ** -16)), (512, np.float32(1.0))):
        ptr = np.array([0, d] + [d] * (n - 1), np.int32)
        ind = np.arange(d, dtype=np.int32)
        val = np.ones(d, np.float32)
        B = np.full((n, 1), 2.0 ** -25, np.float32)
        B[0, 0] = 1.0
        C = oracle.spmm_csr(ptr, ind, val, B)
        assert C[0, 0] == want, (d, C[0, 0])
    # The same row with no segmentation is a single chain.
    ptr = np.array([0, 1024] + [1024] * (n - 1), np.int32)
    C = oracle.spmm_csr(ptr, np.arange(1024, dtype=np.int32), np.ones(1024, np.float32), B,
                        long_row=1 << 30)
    assert C[0, 0] == np.float32(1.0)
