"""Host checks of the synthetic generators that measurements rely on."""

import numpy as np

from chunkedgreedy_amd import synth


def test_rgg_edges_against_brute_force():
    """Every pair of points closer than r is an edge and no other pair is;
    points numbered cell by cell (row-major cells of side >= r)."""
    n, deg, seed = 1500, 9.0, 4
    ptr, ind, val = synth.rgg(n, deg, seed)
    rng = np.random.Generator(np.random.PCG64(seed))
    pts = rng.random((n, 2))
    r = np.sqrt(deg / (np.pi * n))
    g = max(1, int(1.0 / r))
    cell = np.minimum((pts * g).astype(np.int64), g - 1)
    order = np.argsort(cell[:, 1] * g + cell[:, 0], kind="stable")
    pts = pts[order]
    d2 = ((pts[:, None, :] - pts[None, :, :]) ** 2).sum(axis=2)
    want = (d2 < r * r) & ~np.eye(n, dtype=bool)
    got = np.zeros((n, n), bool)
    got[np.repeat(np.arange(n), np.diff(ptr)), ind] = True
    assert np.array_equal(got, want)
    assert (val == 1.0).all()
    assert synth.is_pattern_symmetric(ptr, ind)


def test_chung_lu_reaches_its_mean_degree():
    """Off-diagonal entries per row reach the requested mean (drawn in rounds
    until they do) without overshooting by more than 1 %; every row holds its
    diagonal; values are D^-1/2 (A + I) D^-1/2."""
    n, deg = 20000, 8.0
    ptr, ind, val = synth.chung_lu(n, 2.1, deg, 7)
    rows = np.repeat(np.arange(n), np.diff(ptr))
    off = (rows != ind).sum() / n
    assert deg <= off < deg * 1.01
    assert ((rows == ind).sum()) == n
    assert synth.is_pattern_symmetric(ptr, ind)
    d = np.diff(ptr).astype(np.float64)
    np.testing.assert_allclose(val, (1.0 / np.sqrt(d[rows] * d[ind])).astype(np.float32),
                               rtol=1e-6)


def test_chung_lu_degree_order_is_the_same_graph_relabelled():
    """Without the scramble the graph is the scrambled one relabelled (the
    edges are drawn first, the relabelling last): the same multiset of edges
    seen as (degree of row, degree of column) pairs, and the largest expected
    degrees at the lowest ids."""
    n, deg = 20000, 8.0
    ptr_s, ind_s, _ = synth.chung_lu(n, 2.1, deg, 7)
    ptr_d, ind_d, _ = synth.chung_lu(n, 2.1, deg, 7, scramble=False)
    ds, dd = np.diff(ptr_s), np.diff(ptr_d)

    def degree_pairs(ptr, ind, d):
        rows = np.repeat(np.arange(n), np.diff(ptr))
        return np.sort(d[rows].astype(np.int64) * (n + 1) + d[ind])

    assert np.array_equal(degree_pairs(ptr_s, ind_s, ds), degree_pairs(ptr_d, ind_d, dd))
    assert dd[:100].mean() > 10 * dd.mean()
    assert ds[:100].mean() < 3 * ds.mean()
