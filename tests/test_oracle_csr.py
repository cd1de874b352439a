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


def test_spmm_fmaf_order():
    """Each output is a left-to-right fmaf chain in CSR order: check the
    longest row against exact arithmetic rounded once per step."""
    from fractions import Fraction

    ptr, ind, val = MATS["rmat10"]
    n = ptr.shape[0] - 1
    B = np.random.default_rng(9).standard_normal((n, 3)).astype(np.float32)
    C = oracle.spmm_csr(ptr, ind, val, B)
    r = int(np.argmax(np.diff(ptr)))
    for j in range(3):
        acc = np.float32(0.0)
        for p in range(ptr[r], ptr[r + 1]):
            exact = Fraction(float(val[p])) * Fraction(float(B[ind[p], j])) + Fraction(float(acc))
            acc = round_f32(exact)
        assert C[r, j].view(np.uint32) == acc.view(np.uint32)
