"""CPU oracle for the sporder-csg path -- TEST INFRASTRUCTURE ONLY.

numpy/ctypes front end of ``oracle/csg_oracle.cpp`` (a C++ restatement of the
reference algorithm, each function citing the reference file:line it follows).
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module, and only as the checker or the CPU baseline; the
product path (``chunkedgreedy_amd``) never imports it.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle_csg.so"

_lib = None


class CsgStats(ctypes.Structure):
    """Layout of sporder_csg_stats_t (reference sporder/include/sporder.h:213-222)."""

    _fields_ = [
        ("k_used", ctypes.c_int32),
        ("m_used", ctypes.c_int32),
        ("avg_degree", ctypes.c_double),
        ("avg_edge_weight", ctypes.c_double),
        ("zero_degree_rows", ctypes.c_int32),
        ("chunk_size_used", ctypes.c_int32),
        ("chain_restarts", ctypes.c_int32),
        ("avg_followed_weight", ctypes.c_double),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


def build(force: bool = False) -> Path:
    """Compile the oracle with its Makefile (g++ -fopenmp)."""
    if force or not LIB_PATH.exists():
        subprocess.run(["make", "-s", "-B" if force else "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def _P(t):
    return ctypes.POINTER(t)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        i32, f32, f64, u64, i64 = (ctypes.c_int32, ctypes.c_float, ctypes.c_double,
                                   ctypes.c_uint64, ctypes.c_int64)
        L.oracle_csg_defaults.argtypes = [i32, i32, i32, f32, i32, _P(i32), _P(f32), _P(i32), _P(i32)]
        L.oracle_csg_defaults.restype = None
        L.oracle_csr2csc.argtypes = [i32, i32, _P(i32), _P(i32), _P(i32), _P(i32)]
        L.oracle_csr2csc.restype = None
        L.oracle_chunk_similarity_top_k.argtypes = [i32, i32, i32, f32, _P(i32), _P(i32),
                                                    _P(i32), _P(i32), _P(u64)]
        L.oracle_chunk_similarity_top_k.restype = i32
        L.oracle_sketch_stream.argtypes = [i32, i32, i32, _P(i32), _P(f32), _P(u64)]
        L.oracle_sketch_stream.restype = None
        L.oracle_greedy.argtypes = [i32, i32, i32, _P(u64), _P(i32), _P(i64), _P(i64), _P(f64)]
        L.oracle_greedy.restype = None
        L.oracle_top_k_stats.argtypes = [i32, i32, _P(u64), _P(u64), _P(f64), _P(i32)]
        L.oracle_top_k_stats.restype = None
        L.oracle_chunk_similarity_greedy.argtypes = [i32, i32, _P(i32), _P(i32), i32, i32, f32,
                                                     i32, _P(i32), _P(u64), _P(CsgStats)]
        L.oracle_chunk_similarity_greedy.restype = i32
        L.oracle_reorder.argtypes = [i32, i32, _P(i32), _P(i32), _P(f32), _P(i32), i32,
                                     _P(i32), _P(i32), _P(f32)]
        L.oracle_reorder.restype = None
        L.oracle_spmm_csr.argtypes = [i32, _P(i32), _P(i32), _P(f32), i32, _P(f32), _P(f32),
                                       i32, i32]
        L.oracle_spmm_csr.restype = None
        L.oracle_num_threads.argtypes = []
        L.oracle_num_threads.restype = i32
        L.oracle_set_num_threads.argtypes = [i32]
        L.oracle_set_num_threads.restype = None
        _lib = L
    return _lib


def _ptr(a: np.ndarray, t):
    return a.ctypes.data_as(ctypes.POINTER(t))


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


def num_threads() -> int:
    return int(lib().oracle_num_threads())


def set_num_threads(t: int) -> None:
    lib().oracle_set_num_threads(int(t))


# ---- weighted_index packing (reference sporder/src/common/weighted_index.h:15-27)

def unpack_table(table: np.ndarray):
    """Split a u64 weighted_index table into (int32 index, float32 weight)."""
    t = np.ascontiguousarray(table, dtype=np.uint64)
    idx = (t & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.int32) - np.int32(1)
    w = (t >> np.uint64(32)).astype(np.uint32).view(np.float32)
    return idx.astype(np.int32), w


def pack_table(idx: np.ndarray, w: np.ndarray) -> np.ndarray:
    i = (np.asarray(idx, dtype=np.int64) + 1).astype(np.uint32).astype(np.uint64)
    b = np.asarray(w, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return (b << np.uint64(32)) | i


# ---- algorithm entry points ------------------------------------------------

def csg_defaults(n: int, nnz: int, k: int = 0, oversampling: float = 0.0, chunk_size: int = 0):
    ko, oo, co, mo = ctypes.c_int32(), ctypes.c_float(), ctypes.c_int32(), ctypes.c_int32()
    lib().oracle_csg_defaults(n, nnz, k, oversampling, chunk_size, ctypes.byref(ko),
                              ctypes.byref(oo), ctypes.byref(co), ctypes.byref(mo))
    return ko.value, oo.value, co.value, mo.value


def csr2csc(ptr, ind):
    ptr, ind = _i32(ptr), _i32(ind)
    n = ptr.shape[0] - 1
    nnz = ind.shape[0]
    cptr = np.empty(n + 1, np.int32)
    rind = np.empty(max(nnz, 1), np.int32)
    lib().oracle_csr2csc(n, nnz, _ptr(ptr, ctypes.c_int32), _ptr(ind, ctypes.c_int32),
                         _ptr(cptr, ctypes.c_int32), _ptr(rind, ctypes.c_int32))
    return cptr, rind[:nnz]


def chunk_similarity_top_k(ptr, ind, k: int, chunk_size: int, oversampling: float,
                           is_symmetric: bool = False):
    """n x k u64 weighted_index table of the chunk-restricted sketch."""
    ptr, ind = _i32(ptr), _i32(ind)
    n = ptr.shape[0] - 1
    if is_symmetric:
        cptr, rind = ptr, ind
    else:
        cptr, rind = csr2csc(ptr, ind)
    rind = rind if rind.size else np.zeros(1, np.int32)
    ind_c = ind if ind.size else np.zeros(1, np.int32)
    table = np.empty(max(n * k, 1), np.uint64)
    rc = lib().oracle_chunk_similarity_top_k(n, k, chunk_size, oversampling,
                                             _ptr(ptr, ctypes.c_int32), _ptr(ind_c, ctypes.c_int32),
                                             _ptr(cptr, ctypes.c_int32), _ptr(rind, ctypes.c_int32),
                                             _ptr(table, ctypes.c_uint64))
    if rc < 0:
        raise ValueError(f"oracle rejected arguments (code {rc})")
    return table[: n * k].reshape(n, k)


def sketch_stream(m_capacity: int, k: int, keys, weights) -> np.ndarray:
    keys = _i32(keys)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    out = np.zeros(k, np.uint64)
    kk = keys if keys.size else np.zeros(1, np.int32)
    ww = weights if weights.size else np.zeros(1, np.float32)
    lib().oracle_sketch_stream(m_capacity, k, keys.shape[0], _ptr(kk, ctypes.c_int32),
                               _ptr(ww, ctypes.c_float), _ptr(out, ctypes.c_uint64))
    return out


def greedy(table: np.ndarray, chunk_size: int):
    table = np.ascontiguousarray(table, dtype=np.uint64)
    n, k = table.shape
    order = np.empty(max(n, 1), np.int32)
    r, l, w = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_double()
    t = table if table.size else np.zeros((1, 1), np.uint64)
    lib().oracle_greedy(n, k, chunk_size, _ptr(t, ctypes.c_uint64), _ptr(order, ctypes.c_int32),
                        ctypes.byref(r), ctypes.byref(l), ctypes.byref(w))
    return order[:n], {"restarts": r.value, "links": l.value, "link_weight_sum": w.value}


def top_k_stats(table: np.ndarray):
    table = np.ascontiguousarray(table, dtype=np.uint64)
    n, k = table.shape
    d, w, z = ctypes.c_uint64(), ctypes.c_double(), ctypes.c_int32()
    lib().oracle_top_k_stats(n, k, _ptr(table, ctypes.c_uint64), ctypes.byref(d),
                             ctypes.byref(w), ctypes.byref(z))
    return d.value, w.value, z.value


def chunk_similarity_greedy(ptr, ind, *, is_symmetric=False, k=0, oversampling=0.0,
                            chunk_size=0, return_table=False):
    """Oracle of sporder_chunk_similarity_greedy: (new_order, stats[, table])."""
    ptr, ind = _i32(ptr), _i32(ind)
    n = ptr.shape[0] - 1
    nnz = ind.shape[0]
    k_used, _, _, _ = csg_defaults(n, nnz, k, oversampling, chunk_size)
    order = np.empty(max(n, 1), np.int32)
    stats = CsgStats()
    table = np.empty(max(n * k_used, 1), np.uint64) if return_table else None
    ind_c = ind if ind.size else np.zeros(1, np.int32)
    rc = lib().oracle_chunk_similarity_greedy(
        n, nnz, _ptr(ptr, ctypes.c_int32), _ptr(ind_c, ctypes.c_int32), int(bool(is_symmetric)),
        k, oversampling, chunk_size, _ptr(order, ctypes.c_int32),
        _ptr(table, ctypes.c_uint64) if table is not None else None, ctypes.byref(stats))
    if rc < 0:
        raise ValueError(f"oracle rejected arguments (code {rc})")
    out = (order[:n], stats.as_dict())
    if return_table:
        out += (table[: n * k_used].reshape(n, k_used),)
    return out


def chunk_greedy(ptr, ind, *, is_symmetric=False, k=0, oversampling=0.0, chunk_size=0,
                 return_table=False):
    """Oracle of sporder_chunk_greedy (reference sporder/src/cg/chunk_greedy.cu:110-158):
    the global sketch (sporder/src/common/similarity_top_k.cu:10-51, which is the
    chunked sketch with one chunk of n rows), then the per-chunk chain of
    oracle_greedy.  Stats follow sporder/src/cg/stats_collector.cu:45-72:
    cut_weight_fraction = 1 - (weight of table entries inside their row's chunk)
    / (weight of all table entries), clamped to [0, 1].  Returns
    (new_order, stats[, table])."""
    ptr, ind = _i32(ptr), _i32(ind)
    n = ptr.shape[0] - 1
    nnz = ind.shape[0]
    k_used, ovs_used, chunk_used, m_used = csg_defaults(n, nnz, k, oversampling, chunk_size)
    table = chunk_similarity_top_k(ptr, ind, k_used, n, ovs_used, is_symmetric)
    order, ch = greedy(table, chunk_used)
    deg, wsum, zeros = top_k_stats(table)
    idx, w = unpack_table(table)
    valid = idx >= 0
    rows = np.broadcast_to(np.arange(n)[:, None], idx.shape)
    same = valid & (idx // chunk_used == rows // chunk_used)
    in_w = float(w[same].astype(np.float64).sum())
    cut = 1.0 - in_w / wsum if wsum > 0 else 0.0
    stats = {"k_used": k_used, "m_used": m_used,
             "avg_degree": deg / n, "avg_edge_weight": wsum / deg if deg > 0 else 0.0,
             "zero_degree_rows": zeros, "chunk_size_used": chunk_used,
             "chain_restarts": ch["restarts"],
             "avg_followed_weight": ch["link_weight_sum"] / ch["links"] if ch["links"] else 0.0,
             "cut_weight_fraction": min(1.0, max(0.0, cut))}
    out = (order, stats)
    if return_table:
        out += (table,)
    return out


def count_pillars(ptr, ind, height: int) -> int:
    """Oracle of sporder_count_pillars (reference sporder/src/count_pillars.cu:11-85):
    the number of distinct (row // height, column) pairs over all nonzeros.
    Pinned by closed forms (height 1 with distinct columns per row gives nnz,
    height >= n gives the number of distinct columns) and brute-force sets
    (tests/test_oracle_quality.py)."""
    ptr, ind = _i32(ptr), _i32(ind)
    n = ptr.shape[0] - 1
    if height < 1:
        raise ValueError("height must be >= 1")
    rows = np.repeat(np.arange(n, dtype=np.int64), np.diff(ptr))
    keys = (rows // height) * np.int64(n) + ind.astype(np.int64)
    return int(np.unique(keys).size)


def quality_metrics(rows, cols, n: int, mu: int = 16, nu: int = 8) -> dict:
    """Structural reordering-quality metrics of a pattern given as COO
    (reference experiments/quality_metrics.py:36-57):
      pillars   = distinct (row // mu, column) pairs;
      tc_blocks = sum over row windows of ceil(pillars_in_window / nu);
      bandwidth = max |i - j|;
      profile   = sum over nonempty rows of max(0, i - min column);
      log_gap   = mean over nonzeros of log2(gap + 1), gaps between consecutive
                  sorted columns of a row, the first measured from the row index.
    Pinned by closed forms on identity, band and dense-block patterns
    (tests/test_oracle_quality.py)."""
    rows = np.asarray(rows, np.int64)
    cols = np.asarray(cols, np.int64)
    order = np.lexsort((cols, rows))
    r, c = rows[order], cols[order]
    win = r // mu
    uk = np.unique(win * n + c)
    per_win = np.bincount(uk // n)
    first = np.ones(r.size, dtype=bool)
    first[1:] = r[1:] != r[:-1]
    gaps = np.empty(r.size, dtype=np.int64)
    gaps[1:] = c[1:] - c[:-1]
    gaps[first] = np.abs(c[first] - r[first])
    return {"pillars": int(uk.size),
            "tc_blocks": int(np.sum((per_win + nu - 1) // nu)),
            "bandwidth": int(np.max(np.abs(r - c))) if r.size else 0,
            "profile": int(np.sum(np.maximum(0, r[first] - c[first]))),
            "log_gap": float(np.log2(gaps + 1).sum() / r.size) if r.size else 0.0}


def reorder_bench_metrics(ptr, ind, tc_h: int = 16, tc_w: int = 8) -> dict:
    """The structure columns of the reorder-bench CSV (reference
    spmatkit/spmatkit.py:1704-1717 bandwidth/profile as the per-row maximum of
    |i - j| (max and sum over nonempty rows), :1974-1995 windows of tc_h rows
    and ceil(distinct columns / tc_w) tiles, :2052-2060 the fill rate).
    Pinned by closed forms (tests/test_oracle_quality.py)."""
    ptr, ind = _i32(ptr), _i32(ind)
    n = ptr.shape[0] - 1
    nnz = ind.shape[0]
    out = {"tc_h": tc_h, "tc_w": tc_w}
    if nnz == 0:
        out.update(bandwidth=0, profile=0, tc_num=0, tc_fill_rate=float("nan"))
        return out
    rows = np.repeat(np.arange(n, dtype=np.int64), np.diff(ptr))
    dist = np.abs(rows - ind.astype(np.int64))
    row_max = np.zeros(n, np.int64)
    np.maximum.at(row_max, rows, dist)
    nonempty = np.diff(ptr) > 0
    out["bandwidth"] = int(row_max.max())
    out["profile"] = int(row_max[nonempty].sum())
    uk = np.unique((rows // tc_h) * n + ind.astype(np.int64))
    per_win = np.bincount(uk // n)
    tc_num = int(np.sum((per_win + tc_w - 1) // tc_w))
    out["tc_num"] = tc_num
    out["tc_fill_rate"] = nnz / (tc_num * tc_h * tc_w) if tc_num else float("nan")
    return out


def reorder(ptr, ind, new_order, val=None, symmetric=False):
    ptr, ind, new_order = _i32(ptr), _i32(ind), _i32(new_order)
    n = ptr.shape[0] - 1
    nnz = ind.shape[0]
    ptr_new = np.empty(n + 1, np.int32)
    ind_new = np.empty(max(nnz, 1), np.int32)
    val_new = None
    vp = None
    if val is not None:
        val = np.ascontiguousarray(val, dtype=np.float32)
        val_new = np.empty(max(nnz, 1), np.float32)
        vp = _ptr(val if val.size else np.zeros(1, np.float32), ctypes.c_float)
    ind_c = ind if ind.size else np.zeros(1, np.int32)
    no = new_order if new_order.size else np.zeros(1, np.int32)
    lib().oracle_reorder(n, nnz, _ptr(ptr, ctypes.c_int32), _ptr(ind_c, ctypes.c_int32), vp,
                         _ptr(no, ctypes.c_int32), 1 if symmetric else 0,
                         _ptr(ptr_new, ctypes.c_int32), _ptr(ind_new, ctypes.c_int32),
                         _ptr(val_new, ctypes.c_float) if val_new is not None else None)
    if val is None:
        return ptr_new, ind_new[:nnz]
    return ptr_new, ind_new[:nnz], val_new[:nnz]


# The HIP library's stated SpMM order (include/sporder.h SPORDER_SPMM_LONG_ROW,
# SPORDER_SPMM_SEGMENT): rows longer than LONG_ROW are summed in segments.
SPMM_LONG_ROW = 512
SPMM_SEGMENT = 512


def spmm_csr(ptr, ind, val, B, long_row=SPMM_LONG_ROW, seg_len=SPMM_SEGMENT) -> np.ndarray:
    """C = A @ B in the stated order: rows of at most long_row nonzeros as one
    fmaf chain from 0.0f in CSR order; longer rows as chains over segments of
    seg_len nonzeros added left to right."""
    ptr, ind = _i32(ptr), _i32(ind)
    val = np.ascontiguousarray(val, dtype=np.float32)
    B = np.ascontiguousarray(B, dtype=np.float32)
    n = ptr.shape[0] - 1
    N = B.shape[1]
    C = np.empty((n, N), np.float32)
    ind_c = ind if ind.size else np.zeros(1, np.int32)
    val_c = val if val.size else np.zeros(1, np.float32)
    lib().oracle_spmm_csr(n, _ptr(ptr, ctypes.c_int32), _ptr(ind_c, ctypes.c_int32),
                          _ptr(val_c, ctypes.c_float), N, _ptr(B, ctypes.c_float),
                          _ptr(C, ctypes.c_float), int(long_row), int(seg_len))
    return C


__all__ = [
    "CsgStats", "build", "lib", "num_threads", "set_num_threads", "unpack_table",
    "pack_table", "csg_defaults", "csr2csc", "chunk_similarity_top_k", "sketch_stream",
    "greedy", "top_k_stats", "chunk_similarity_greedy", "chunk_greedy", "reorder", "spmm_csr",
    "count_pillars", "quality_metrics", "reorder_bench_metrics",
]

if os.environ.get("SPORDER_ORACLE_THREADS"):
    set_num_threads(int(os.environ["SPORDER_ORACLE_THREADS"]))
