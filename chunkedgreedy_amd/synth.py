"""Seeded synthetic CSR generators for the benchmark configurations.

The reference ships no generators for these inputs (its experiments read
SuiteSparse files), so the shapes follow the configuration text:

  C1 planted(n=20_000, blocks=256, nnz/row=10)          CPU plumbing case
  C2 planted(n=1_048_576, blocks=16_384, nnz/row=16)    headline workload
  C3 rmat(scale=22, edge_factor=16, a,b,c,d=.57,.19,.19,.05), symmetrized,
     deduplicated, no self loops, values 1/deg(row)
  C4 stencil7(160), diagonal 6 / off-diagonal -1, random symmetric permutation
  C5 chung_lu(n=2_449_029, exponent=2.1, avg degree 25), symmetric, with self
     loops, values of D^-1/2 (A+I) D^-1/2

Every generator returns (ptr int32[n+1], ind int32[nnz], val float32[nnz]) with
column indices sorted and distinct within each row, from numpy's PCG64 seeded
by `seed`.  The same seed gives the same matrix on every host.
"""

from __future__ import annotations

import numpy as np

Csr = tuple[np.ndarray, np.ndarray, np.ndarray]


def _rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def _coo_to_csr(n: int, rows: np.ndarray, cols: np.ndarray, vals: np.ndarray) -> Csr:
    # Stable sort by (row, column) on one int64 key: the order np.lexsort gives.
    order = np.argsort(rows.astype(np.int64) * n + cols, kind="stable")
    rows, cols, vals = rows[order], cols[order], vals[order]
    counts = np.bincount(rows, minlength=n)
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(counts, out=ptr[1:])
    return ptr.astype(np.int32), cols.astype(np.int32), vals.astype(np.float32)


def _sort_rows(ptr: np.ndarray, ind: np.ndarray, val: np.ndarray) -> Csr:
    n = ptr.shape[0] - 1
    rows = np.repeat(np.arange(n, dtype=np.int64), np.diff(ptr.astype(np.int64)))
    order = np.argsort(rows * n + ind, kind="stable")
    return ptr.astype(np.int32), ind[order].astype(np.int32), val[order].astype(np.float32)


def permute(ptr, ind, val, row_perm: np.ndarray | None, col_perm: np.ndarray | None) -> Csr:
    """B[i, j] = A[row_perm[i], col_perm[j]] (new2old permutations); rows
    re-sorted."""
    n = ptr.shape[0] - 1
    ptr64 = ptr.astype(np.int64)
    if row_perm is not None:
        lens = np.diff(ptr64)[row_perm]
        new_ptr = np.zeros(n + 1, np.int64)
        np.cumsum(lens, out=new_ptr[1:])
        src = np.repeat(ptr64[row_perm] - new_ptr[:-1], lens) + np.arange(new_ptr[-1])
        ind = ind[src]
        val = val[src]
        ptr64 = new_ptr
    if col_perm is not None:
        inv = np.empty(n, np.int64)
        inv[col_perm] = np.arange(n)
        ind = inv[ind]
    return _sort_rows(ptr64, ind, val)


def planted(n: int, blocks: int, nnz_per_row: int, seed: int, in_frac: float = 0.8,
            planted_rows: bool = False) -> Csr:
    """Planted-block matrix: row i of block b has round(in_frac*nnz_per_row)
    distinct columns inside b's column range and the rest uniform over all
    columns (all distinct); values U(-1,1); then independent random row and
    column permutations.  With planted_rows the rows keep the planted block
    order (the row permutation is drawn, so the columns are the same, but
    not applied): the blocks' rows are contiguous and share their in-block
    columns, which the column permutation scatters."""
    rng = _rng(seed)
    sizes = np.full(blocks, n // blocks, np.int64)
    sizes[: n % blocks] += 1
    starts = np.zeros(blocks + 1, np.int64)
    np.cumsum(sizes, out=starts[1:])
    row_block = np.repeat(np.arange(blocks), sizes)
    bs = starts[row_block]
    bl = sizes[row_block]
    n_in = int(round(in_frac * nnz_per_row))
    n_out = nnz_per_row - n_in
    width = int(sizes.max())
    cols = np.empty((n, nnz_per_row), np.int64)
    step = 1 << 18
    for r0 in range(0, n, step):
        r1 = min(n, r0 + step)
        keys = rng.random((r1 - r0, width), dtype=np.float32)
        keys[np.arange(width)[None, :] >= bl[r0:r1, None]] = 2.0
        pick = np.argpartition(keys, n_in - 1, axis=1)[:, :n_in]
        cols[r0:r1, :n_in] = bs[r0:r1, None] + pick
    if n_out:
        cols[:, n_in:] = rng.integers(0, n, size=(n, n_out))
        # Resample uniform columns that collide with another column of the row.
        while True:
            srt = np.sort(cols, axis=1)
            dup_rows = np.nonzero((srt[:, 1:] == srt[:, :-1]).any(axis=1))[0]
            if dup_rows.size == 0:
                break
            cols[dup_rows, n_in:] = rng.integers(0, n, size=(dup_rows.size, n_out))
    vals = rng.uniform(-1.0, 1.0, size=(n, nnz_per_row)).astype(np.float32)
    row_perm = rng.permutation(n)
    col_perm = rng.permutation(n)
    if planted_rows:
        row_perm = np.arange(n)
    # Every row has the same length, so the permutations and the per-row sort
    # work on the dense (n, nnz_per_row) layout.
    inv = np.empty(n, np.int64)
    inv[col_perm] = np.arange(n)
    cols = inv[cols[row_perm]]
    vals = vals[row_perm]
    order = np.argsort(cols, axis=1, kind="stable")
    cols = np.take_along_axis(cols, order, axis=1)
    vals = np.take_along_axis(vals, order, axis=1)
    ptr = np.arange(n + 1, dtype=np.int64) * nnz_per_row
    return ptr.astype(np.int32), cols.reshape(-1).astype(np.int32), vals.reshape(-1)


def config1(seed: int = 1) -> Csr:
    return planted(20_000, 256, 10, seed)


def config2(seed: int = 2, n: int = 1_048_576, blocks: int = 16_384,
            planted_rows: bool = False) -> Csr:
    return planted(n, blocks, 16, seed, planted_rows=planted_rows)


def rmat(scale: int, edge_factor: int, seed: int, a=0.57, b=0.19, c=0.19) -> Csr:
    """R-MAT graph (Chakrabarti, Zhan, Faloutsos 2004): edge_factor * 2^scale
    edges, each placed by `scale` independent quadrant choices; symmetrized,
    deduplicated, self loops removed; values 1/deg(row)."""
    rng = _rng(seed)
    n = 1 << scale
    m = edge_factor * n
    keys = []
    step = 1 << 22
    for e0 in range(0, m, step):
        cnt = min(step, m - e0)
        u = np.zeros(cnt, np.int64)
        v = np.zeros(cnt, np.int64)
        for _ in range(scale):
            r = rng.random(cnt)
            down = r >= a + b          # quadrants c, d
            right = ((r >= a) & (r < a + b)) | (r >= a + b + c)  # b, d
            u = (u << 1) | down
            v = (v << 1) | right
        keep = u != v
        u, v = u[keep], v[keep]
        keys.append(u * n + v)
        keys.append(v * n + u)
    k = np.unique(np.concatenate(keys))
    rows = k // n
    cols = k % n
    counts = np.bincount(rows, minlength=n)
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(counts, out=ptr[1:])
    deg = np.maximum(counts, 1).astype(np.float32)
    val = (1.0 / deg)[rows].astype(np.float32)
    return ptr.astype(np.int32), cols.astype(np.int32), val


def config3(seed: int = 3, scale: int = 22) -> Csr:
    return rmat(scale, 16, seed)


def stencil7(g: int, seed: int, scramble: bool = True) -> Csr:
    """7-point stencil on a g^3 grid (6 on the diagonal, -1 off it), with a
    random symmetric permutation P A P^T."""
    n = g ** 3
    idx = np.arange(n, dtype=np.int64)
    x, y, z = idx % g, (idx // g) % g, idx // (g * g)
    rows, cols, vals = [idx], [idx], [np.full(n, 6.0, np.float32)]
    for d, coord in ((1, x), (g, y), (g * g, z)):
        m = coord < g - 1
        rows += [idx[m], idx[m] + d]
        cols += [idx[m] + d, idx[m]]
        vals += [np.full(int(m.sum()), -1.0, np.float32)] * 2
    ptr, ind, val = _coo_to_csr(n, np.concatenate(rows), np.concatenate(cols),
                                np.concatenate(vals))
    if scramble:
        p = _rng(seed).permutation(n)
        ptr, ind, val = permute(ptr, ind, val, p, p)
    return ptr, ind, val


def config4(seed: int = 4, g: int = 160) -> Csr:
    return stencil7(g, seed)


def _alias_table(w: np.ndarray):
    """Walker's alias table (Vose's construction) for sampling index i with
    probability w[i] / sum(w) in O(1): draw i uniformly, keep it with
    probability prob[i], else take alias[i]."""
    n = w.shape[0]
    p = (w * (n / w.sum())).tolist()
    prob = [1.0] * n
    alias = list(range(n))
    small = [i for i in range(n) if p[i] < 1.0]
    large = [i for i in range(n) if p[i] >= 1.0]
    while small and large:
        s = small.pop()
        g = large.pop()
        prob[s] = p[s]
        alias[s] = g
        p[g] = p[g] + p[s] - 1.0
        (small if p[g] < 1.0 else large).append(g)
    return np.array(prob), np.array(alias, np.int64)


def chung_lu(n: int, exponent: float, avg_degree: float, seed: int,
             scramble: bool = True) -> Csr:
    """Chung-Lu graph with expected degrees w_i proportional to
    (i + 1)^(-1/(exponent-1)): edges with both endpoints drawn proportional to
    w, symmetrized and deduplicated, drawn in rounds until the mean number of
    distinct neighbours (self loops excluded) reaches `avg_degree` (the hubs
    draw many duplicates, so n*avg_degree/2 draws alone fall short); then the
    identity added and values D^-1/2 (A + I) D^-1/2.  With `scramble` (the
    default) vertex ids are a random permutation of the expected-degree order;
    without it vertex i is the i-th largest expected degree (the same graph,
    relabelled: the edges are drawn first, the relabelling last)."""
    rng = _rng(seed)
    w = (np.arange(n, dtype=np.float64) + 1.0) ** (-1.0 / (exponent - 1.0))
    prob, alias = _alias_table(w)
    target = int(round(n * avg_degree))  # directed off-diagonal entries
    k = np.zeros(0, np.int64)
    m = int(n * avg_degree / 2)
    step = 1 << 22

    def draw(cnt):
        i = rng.integers(0, n, cnt)
        return np.where(rng.random(cnt) < prob[i], i, alias[i])

    while True:
        keys = [k]
        for e0 in range(0, m, step):
            cnt = min(step, m - e0)
            u = draw(cnt)
            v = draw(cnt)
            keep = u != v
            u, v = u[keep], v[keep]
            keys += [u * n + v, v * n + u]
        before = k.shape[0]
        k = np.unique(np.concatenate(keys))
        if k.shape[0] >= target:
            break
        # Draw the shortfall again, scaled by this round's yield of new
        # entries per draw (it falls as the hubs fill up).
        per_draw = max((k.shape[0] - before) / m, 1e-3)
        m = max(1024, int((target - k.shape[0]) / per_draw * 1.05))
    k = np.union1d(k, np.arange(n, dtype=np.int64) * (n + 1))  # self loops
    # Scramble vertex ids so that degree does not follow the index.
    p = rng.permutation(n) if scramble else np.arange(n, dtype=np.int64)
    rows, cols = p[k // n], p[k % n]
    deg = np.bincount(rows, minlength=n).astype(np.float64)
    dinv = 1.0 / np.sqrt(deg)
    vals = (dinv[rows] * dinv[cols]).astype(np.float32)
    return _coo_to_csr(n, rows, cols, vals)


def config5(seed: int = 5, n: int = 2_449_029, scramble: bool = True) -> Csr:
    return chung_lu(n, 2.1, 25.0, seed, scramble=scramble)


def rgg(n: int, avg_degree: float, seed: int) -> Csr:
    """Random geometric graph: n points uniform in the unit square, an edge
    between two points closer than r = sqrt(avg_degree / (pi n)) (no self
    loops), values 1.  Points are numbered cell by cell over a grid of cells
    of side >= r (row-major cells, points in a cell in draw order), so
    neighbours are near in index: a stand-in with the locality of the
    rgg_n_2_20 graphs the reference's reorder benchmark reports."""
    rng = _rng(seed)
    r = float(np.sqrt(avg_degree / (np.pi * n)))
    g = max(1, int(1.0 / r))
    pts = rng.random((n, 2))
    cell = np.minimum((pts * g).astype(np.int64), g - 1)
    cid = cell[:, 1] * g + cell[:, 0]
    order = np.argsort(cid, kind="stable")
    pts, cell, cid = pts[order], cell[order], cid[order]
    cstart = np.searchsorted(cid, np.arange(g * g + 1))
    rows, cols = [], []
    for dy in (-1, 0, 1):
        for dx in (-1, 0, 1):
            ox, oy = cell[:, 0] + dx, cell[:, 1] + dy
            ok = (ox >= 0) & (ox < g) & (oy >= 0) & (oy < g)
            src = np.nonzero(ok)[0]
            nb = oy[src] * g + ox[src]
            lo, hi = cstart[nb], cstart[nb + 1]
            cnt = hi - lo
            a = np.repeat(src, cnt)
            b = np.repeat(lo - np.cumsum(np.concatenate([[0], cnt[:-1]])), cnt) + np.arange(cnt.sum())
            d = pts[a] - pts[b]
            keep = (a != b) & ((d * d).sum(axis=1) < r * r)
            rows.append(a[keep])
            cols.append(b[keep])
    rows, cols = np.concatenate(rows), np.concatenate(cols)
    return _coo_to_csr(n, rows, cols, np.ones(rows.shape[0], np.float32))


def band(n: int, half_width: int = 2) -> Csr:
    """Symmetric band pattern |i - j| <= half_width, values 1 (the reference's
    smoke matrix, sporder/tests/smoke.c:58-70, with half_width 2)."""
    rows, cols = [], []
    for d in range(-half_width, half_width + 1):
        i = np.arange(max(0, -d), min(n, n - d), dtype=np.int64)
        rows.append(i)
        cols.append(i + d)
    r = np.concatenate(rows)
    c = np.concatenate(cols)
    return _coo_to_csr(n, r, c, np.ones(r.shape[0], np.float32))


def dense_groups(n: int = 8192, chunk: int = 1024, seed: int = 5) -> Csr:
    """Two dense row groups per chunk of `chunk` rows, every other row alone:
    rows 0..71 of a chunk hold each of the chunk's columns 0..23 with
    probability 0.7 (about 70 in-chunk similar rows each, past one wave's 64
    lanes), rows 100..139 each of columns 30..45 with probability 0.6 and
    now and then one of the first group's columns (about 40); the rest hold
    only their diagonal.  With k >= 72 the chain walks rows of both lengths in
    one chunk.  Values 1."""
    rng = _rng(seed)
    rows, cols = [], []
    for r in range(n):
        base = (r // chunk) * chunk
        o = r - base
        if o < 72:
            c = base + np.nonzero(rng.random(24) < 0.7)[0]
        elif 100 <= o < 140:
            c = base + 30 + np.nonzero(rng.random(16) < 0.6)[0]
            if rng.random() < 0.1:
                c = np.append(c, base + int(rng.integers(0, 24)))
        else:
            c = np.array([r])
        c = np.unique(c[c < n]) if c.size else np.array([r])
        rows.append(np.full(c.size, r, np.int64))
        cols.append(c.astype(np.int64))
    r = np.concatenate(rows)
    c = np.concatenate(cols)
    return _coo_to_csr(n, r, c, np.ones(r.shape[0], np.float32))


def is_pattern_symmetric(ptr, ind) -> bool:
    """Pattern equals its transpose (the harness test of
    bench/reorder/reorder_bench/loader.py:86-88 on the pattern)."""
    import scipy.sparse as sp

    n = ptr.shape[0] - 1
    a = sp.csr_matrix((np.ones(ind.shape[0], np.int8), ind, ptr), shape=(n, n))
    return (a != a.T).nnz == 0


CONFIGS = {
    "C1": config1,
    "C2": config2,
    "C3": config3,
    "C4": config4,
    "C5": config5,
}

# Inputs whose rows carry locality inside each chunk (the reorder benchmark's
# SuiteSparse and DIMACS matrices do; C2 and C4 as configured are scrambled, so
# their chunk-restricted candidate streams are nearly empty): C2 with its rows
# in planted block order, C4 in natural grid order, a random geometric graph of
# 2^20 points with mean degree 13, and C5 with vertices in expected-degree
# order (hubs first, the order a degree-sorted graph file has).
LOCALITY = {
    "C2r": lambda: config2(planted_rows=True),
    "C4n": lambda: stencil7(160, 4, scramble=False),
    "RGG20": lambda: rgg(1 << 20, 13.0, 20),
    "C5d": lambda: config5(scramble=False),
}
