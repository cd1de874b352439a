"""sporder -- sparse-matrix row reordering on AMD Instinct MI355X.

Drop-in for the reference's Python package (sporder/python/sporder/__init__.py
of Siaaa-3/ChunkedGreedy): the same function names, keyword-only arguments,
defaults and return conventions, backed by libsporder_hip.so.  Arrays are
torch tensors on a ROCm GPU (int32 CSR ``ptr``/``ind``); results come back
as torch tensors on the same device.

Provided: chunk_similarity_greedy (sporder-csg), chunk_greedy (sporder-cg),
reorder, count_pillars, similarity_graph, bench_cusparse_spmm, plus spmm_csr
and chunk_similarity_top_k (new).  hierarchical_matching and
similarity_graph_exact exist for import compatibility and raise
NotImplementedError.
"""

from __future__ import annotations

from ._sporder import Context
from ._sporder import bench_cusparse_spmm as _bench_cusparse_spmm
from ._sporder import chunk_greedy as _chunk_greedy
from ._sporder import chunk_similarity_greedy as _chunk_similarity_greedy
from ._sporder import chunk_similarity_top_k as _chunk_similarity_top_k
from ._sporder import count_pillars as _count_pillars
from ._sporder import hierarchical_matching as _hierarchical_matching
from ._sporder import reorder as _reorder
from ._sporder import similarity_graph as _similarity_graph
from ._sporder import similarity_graph_exact as _similarity_graph_exact
from ._sporder import spmm_csr as _spmm_csr
from ._sporder import spmm_csr_noalloc as _spmm_csr_noalloc
from ._sporder import spmm_csr_scaled as _spmm_csr_scaled
from ._sporder import SpmmPlan

__all__ = [
    "bench_cusparse_spmm",
    "Context",
    "chunk_greedy",
    "chunk_similarity_greedy",
    "chunk_similarity_top_k",
    "count_pillars",
    "hierarchical_matching",
    "reorder",
    "similarity_graph",
    "similarity_graph_exact",
    "spmm_csr",
    "spmm_csr_noalloc",
    "spmm_csr_scaled",
    "spmm_plan",
    "SpmmPlan",
]


def _asarray_like(array, reference):
    """Return `array` in the framework of `reference` (reference
    sporder/python/sporder/__init__.py:28-39); results here are torch tensors
    already, converted through DLPack for other frameworks."""
    root = type(reference).__module__.partition(".")[0]
    if root == "torch":
        return array
    if root == "cupy":  # pragma: no cover - CuPy is not part of this image
        import cupy

        return cupy.from_dlpack(array)
    return array


def _pack(first, timing, stats, with_timing, with_stats):
    result = first if isinstance(first, tuple) else (first,)
    if with_timing:
        result += (timing,)
    if with_stats:
        result += (stats,)
    return result


def chunk_similarity_greedy(ptr, ind, *, is_symmetric=False, k=0, oversampling=0.0,
                            chunk_size=0, with_timing=False, with_stats=False, ctx=None):
    """Chunked Greedy row ordering (sporder-csg).

    Rows are cut into aligned chunks of ``chunk_size`` rows.  Within each
    chunk every row gets its top-k Dice neighbours from a space-saving sketch
    (capacity 32*ceil(int(k*oversampling)/32)), and a greedy nearest-neighbour
    chain, restarting at the lowest unvisited row, orders the chunk.

    Arguments:
        ptr, ind: int32 GPU arrays, CSR row pointers (n+1) and columns (nnz)
        is_symmetric: the pattern equals its transpose (skips the transpose)
        k: neighbours per row (0 = clamp(nnz // n, 16, 256))
        oversampling: sketch oversampling (0 = 4.0); int(k*oversampling) <= 512
        chunk_size: rows per chunk (0 = 1024)
        with_timing: also return {wall_ms, csr2csc_ms, similarity_ms,
            chunk_greedy_ms}
        with_stats: also return {k_used, m_used, avg_degree, avg_edge_weight,
            zero_degree_rows, chunk_size_used, chain_restarts,
            avg_followed_weight}
        ctx: Context, or None for the shared default context

    Returns new_order (int32, new2old), followed by timing and/or stats when
    requested.  Reference: sporder/python/sporder/__init__.py:380-424.
    """
    new_order, timing, stats = _chunk_similarity_greedy(
        ptr, ind, is_symmetric=is_symmetric, k=k, oversampling=oversampling,
        chunk_size=chunk_size, with_timing=with_timing, with_stats=with_stats, ctx=ctx)
    result = _pack(_asarray_like(new_order, ptr), timing, stats, with_timing, with_stats)
    return result if len(result) > 1 else result[0]


def reorder(ptr, ind, new_order, *, val=None, symmetric=False, ctx=None):
    """Permute a CSR matrix: row p of the result is row new_order[p]; with
    symmetric=True columns are renumbered by the same permutation (P A P^T)
    and each row re-sorted.  Returns (ptr_new, ind_new[, val_new]).
    Reference: sporder/python/sporder/__init__.py:113-149."""
    if val is not None:
        ptr_new, ind_new, val_new = _reorder(ptr, ind, val=val, new_order=new_order,
                                             symmetric=symmetric, ctx=ctx)
        return (_asarray_like(ptr_new, ptr), _asarray_like(ind_new, ptr),
                _asarray_like(val_new, ptr))
    ptr_new, ind_new = _reorder(ptr, ind, val=None, new_order=new_order,
                                symmetric=symmetric, ctx=ctx)
    return _asarray_like(ptr_new, ptr), _asarray_like(ind_new, ptr)


def bench_cusparse_spmm(ptr, ind, cols, *, warmup=3, repeat=10, seed=0, ctx=None):
    """Mean milliseconds per SpMM launch on the pattern with U(0,1] values and a
    ``cols``-wide dense B generated from ``seed`` (this build times its own
    HIP CSR SpMM).  Reference: sporder/python/sporder/__init__.py:175-197."""
    return _bench_cusparse_spmm(ptr, ind, cols, warmup=warmup, repeat=repeat, seed=seed,
                                ctx=ctx)


def similarity_graph(ptr, ind, *, is_symmetric=False, k=0, oversampling=0.0,
                     with_timing=False, with_stats=False, ctx=None):
    """Global top-k Dice similarity graph from the space-saving sketch.

    Returns (indices, weights) as n x k arrays (k = 0 picks
    clamp(2*nnz//n, 16, 32)); unused entries are (-1, 0.0).  Timing/stats
    dicts are appended when requested.
    Reference: sporder/python/sporder/__init__.py:200-259."""
    idx, wgt, timing, stats = _similarity_graph(
        ptr, ind, is_symmetric=is_symmetric, k=k, oversampling=oversampling,
        with_timing=with_timing, with_stats=with_stats, ctx=ctx)
    n = ptr.shape[0] - 1
    if k <= 0:
        nnz = ind.shape[0] if hasattr(ind, "shape") else len(ind)
        k = min(32, max(16, 2 * nnz // n))
    idx = _asarray_like(idx, ptr).reshape(n, k)
    wgt = _asarray_like(wgt, ptr).reshape(n, k)
    return _pack((idx, wgt), timing, stats, with_timing, with_stats)


def chunk_similarity_top_k(ptr, ind, *, k, oversampling, chunk_size, is_symmetric=False,
                           ctx=None):
    """(new) The csg sketch table: (indices, weights), n x k, each row's top-k
    neighbours inside its chunk.  All parameters must be resolved (> 0)."""
    return _chunk_similarity_top_k(ptr, ind, k, oversampling, chunk_size,
                                   is_symmetric=is_symmetric, ctx=ctx)


def spmm_plan(ptr, ind, *, ctx=None):
    """(new) Analyse a CSR pattern for the planned SpMM (the harness's untimed
    prepare step): a 64-row tile whose 8-row blocks hold at most half as many
    distinct columns as nonzeros is "blocked", and the planned SpMM loads each
    such column's row of B once per block for every row of the block that
    holds it.  Returns an SpmmPlan whose ``info`` dict counts the tiles, the
    blocked tiles, their rows and nonzeros, and the (column, row mask)
    entries."""
    return SpmmPlan(ptr, ind, ctx=ctx)


def spmm_csr(ptr, ind, val, B, *, out=None, algo="row_split", ctx=None, plan=None):
    """(new) C = A @ B for CSR A (values ``val``) and row-major dense B.

    algo "row_split" follows the stated order of include/sporder.h: a row of
    at most 512 nonzeros is one fmaf chain in CSR order, a longer row is summed
    in 512-nonzero segments added left to right (bit-reproducible);
    "merge_path" splits the nonzeros evenly across waves and adds the partial
    sums of cut rows with atomics.  With ``plan`` (spmm_plan of this pattern)
    the blocked tiles load each distinct column's B row once per 8-row block
    and the others run the row-split; the result equals "row_split" bit for
    bit.  Returns (C, kernel_ms)."""
    return _spmm_csr(ptr, ind, val, B, out=out, algo=algo, ctx=ctx, plan=plan)


def spmm_csr_scaled(ptr, ind, val, B, *, row_scale=None, col_scale=None, nz_col_scale=None,
                    out=None, ctx=None):
    """(new) C = diag(row_scale) A diag(col_scale) B in the row-split's stated
    order, with each gathered B row multiplied by its column's scale and each
    finished row by its row scale (one fp32 multiply per element each): equal,
    bit for bit, to ``row_scale[:, None] * spmm_csr(ptr, ind, val,
    col_scale[:, None] * B)[0]`` without the two elementwise passes (a GCN's
    D^-1/2 A D^-1/2, applied around the SpMM as experiments/e2e_gcn.py:117-123
    does).  The kernels read the column scales per nonzero, col_scale[ind]:
    give them as ``nz_col_scale`` to reuse them across calls on one pattern.
    Either scale may be None.  Returns (C, kernel_ms)."""
    return _spmm_csr_scaled(ptr, ind, val, B, row_scale=row_scale, col_scale=col_scale,
                            nz_col_scale=nz_col_scale, out=out, ctx=ctx)


def spmm_csr_noalloc(ptr, ind, val, B, *, out, ctx=None):
    """(new) spmm_csr's row-split into the caller's ``out`` with no device
    allocation by the library: its long-row scratch is a 64 MiB static device
    array per GPU, shared by every call on that GPU (overlapping calls race).
    Bit-identical to spmm_csr(algo="row_split").  Raises ValueError when the
    matrix's long rows need more scratch than that.  Returns ``out``."""
    return _spmm_csr_noalloc(ptr, ind, val, B, out, ctx=ctx)


def hierarchical_matching(ptr, ind, *, is_symmetric=False, num_levels=1, k=0,
                          oversampling=0.0, max_rounds=0, with_timing=False,
                          with_stats=False, ctx=None):
    """Not part of this build (reference __init__.py:42-110)."""
    return _hierarchical_matching(ptr, ind)


def chunk_greedy(ptr, ind, *, is_symmetric=False, k=0, oversampling=0.0, chunk_size=0,
                 with_timing=False, with_stats=False, ctx=None):
    """Chunked greedy seriation on the global similarity graph (sporder-cg,
    "CG w/o Stage 1").

    Every row gets its top-k Dice neighbours from a space-saving sketch over
    the whole matrix (capacity 32*ceil(int(k*oversampling)/32)); rows are then
    cut into aligned chunks of ``chunk_size`` and a greedy nearest-neighbour
    chain, following only neighbours inside the chunk and restarting at the
    lowest unvisited row, orders each chunk.

    Arguments:
        ptr, ind: int32 GPU arrays, CSR row pointers (n+1) and columns (nnz)
        is_symmetric: the pattern equals its transpose (skips the transpose)
        k: neighbours per row (0 = clamp(nnz // n, 16, 256))
        oversampling: sketch oversampling (0 = 4.0); int(k*oversampling) <= 512
        chunk_size: rows per chunk (0 = 1024)
        with_timing: also return {wall_ms, csr2csc_ms, similarity_ms,
            chunk_greedy_ms}
        with_stats: also return {k_used, m_used, avg_degree, avg_edge_weight,
            zero_degree_rows, chunk_size_used, chain_restarts,
            avg_followed_weight, cut_weight_fraction}; cut_weight_fraction is
            the top-k edge weight leaving its row's chunk over the total
        ctx: Context, or None for the shared default context

    Returns new_order (int32, new2old), followed by timing and/or stats when
    requested.  Reference: sporder/python/sporder/__init__.py:311-377.
    """
    new_order, timing, stats = _chunk_greedy(
        ptr, ind, is_symmetric=is_symmetric, k=k, oversampling=oversampling,
        chunk_size=chunk_size, with_timing=with_timing, with_stats=with_stats, ctx=ctx)
    result = _pack(_asarray_like(new_order, ptr), timing, stats, with_timing, with_stats)
    return result if len(result) > 1 else result[0]


def count_pillars(ptr, ind, height, *, ctx=None):
    """Count nonzero columns over consecutive row windows.

    Rows are grouped into ceil(n / height) consecutive windows of ``height``
    rows (the last may be shorter).  A pillar is a column holding at least one
    nonzero inside a window; the total over all windows is the column-tile
    count of a blocked SpMM with tile width 1, the quantity row reordering
    tries to reduce.  Column indices need not be sorted or distinct.

    Arguments:
        ptr, ind: int32 GPU arrays, CSR row pointers (n+1) and columns (nnz)
        height: row window height, >= 1
        ctx: Context, or None for the shared default context

    Returns the pillar total (int).  Reference:
    sporder/python/sporder/__init__.py:152-172.
    """
    return _count_pillars(ptr, ind, height, ctx=ctx)


def similarity_graph_exact(ptr, ind, *, is_symmetric=False, k=0, with_timing=False,
                           with_stats=False, ctx=None):
    """Not part of this build (reference __init__.py:262-308)."""
    return _similarity_graph_exact(ptr, ind)
