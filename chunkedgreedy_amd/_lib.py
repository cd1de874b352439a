"""ctypes view of libsporder_hip.so (the C ABI declared in include/sporder.h).

The library is loaded from the package directory.  A missing library is an
error (no fallback): build it with ``__graft_entry__.build()`` or
``python chunkedgreedy_amd/build.py``.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libsporder_hip.so"

i32 = ctypes.c_int32
i64 = ctypes.c_int64
u64 = ctypes.c_uint64
f32 = ctypes.c_float
f64 = ctypes.c_double
vp = ctypes.c_void_p
P = ctypes.POINTER


class CsgTiming(ctypes.Structure):
    """sporder_csg_timing_t (reference sporder/include/sporder.h:203-208)."""

    _fields_ = [("wall_ms", f64), ("csr2csc_ms", f32), ("similarity_ms", f32),
                ("chunk_greedy_ms", f32)]


class CsgStats(ctypes.Structure):
    """sporder_csg_stats_t (reference sporder/include/sporder.h:213-222)."""

    _fields_ = [("k_used", i32), ("m_used", i32), ("avg_degree", f64),
                ("avg_edge_weight", f64), ("zero_degree_rows", i32),
                ("chunk_size_used", i32), ("chain_restarts", i32),
                ("avg_followed_weight", f64)]


class SpmmPlanInfo(ctypes.Structure):
    """sporder_spmm_plan_info_t (new)."""

    _fields_ = [("tiles", i32), ("blocked_tiles", i32), ("blocked_rows", ctypes.c_int64),
                ("blocked_nnz", ctypes.c_int64), ("entries", ctypes.c_int64)]


class CgTiming(ctypes.Structure):
    """sporder_cg_timing_t (reference sporder/include/sporder.h:128-133)."""

    _fields_ = [("wall_ms", f64), ("csr2csc_ms", f32), ("similarity_ms", f32),
                ("chunk_greedy_ms", f32)]


class CgStats(ctypes.Structure):
    """sporder_cg_stats_t (reference sporder/include/sporder.h:154-167)."""

    _fields_ = [("k_used", i32), ("m_used", i32), ("avg_degree", f64),
                ("avg_edge_weight", f64), ("zero_degree_rows", i32),
                ("chunk_size_used", i32), ("chain_restarts", i32),
                ("avg_followed_weight", f64), ("cut_weight_fraction", f64)]


class SimTiming(ctypes.Structure):
    """sporder_sim_timing_t (reference sporder/include/sporder.h:312-317)."""

    _fields_ = [("wall_ms", f64), ("csr2csc_ms", f32), ("similarity_ms", f32),
                ("unpack_ms", f32)]


class SimStats(ctypes.Structure):
    """sporder_sim_stats_t (reference sporder/include/sporder.h:322-328)."""

    _fields_ = [("k_used", i32), ("m_used", i32), ("avg_degree", f64),
                ("avg_edge_weight", f64), ("zero_degree_rows", i32)]


class HmTiming(ctypes.Structure):
    """sporder_hm_timing_t (reference sporder/include/sporder.h:64-72)."""

    _fields_ = [("wall_ms", f64), ("csr2csc_ms", f32), ("similarity_ms", f32),
                ("matching_ms", f32), ("advance_ms", f32),
                ("matching_per_level_ms", P(f32)), ("advance_per_level_ms", P(f32))]


class HmStats(ctypes.Structure):
    """sporder_hm_stats_t (reference sporder/include/sporder.h:85-94)."""

    _fields_ = [("k_used", i32), ("m_used", i32), ("avg_degree", f64),
                ("avg_edge_weight", f64), ("zero_degree_rows", i32),
                ("level_size", P(i32)), ("matched_pairs", P(i32)), ("rounds", P(i32))]


class Options(ctypes.Structure):
    """sporder_options_t (reference sporder/include/sporder.h:54-58)."""

    _fields_ = [("k", i32), ("oversampling", f32), ("max_rounds", i32)]


REORDER_ROWS = 0
REORDER_SYMMETRIC = 1
SPMM_AUTO = 0
SPMM_ROW_SPLIT = 1
SPMM_MERGE_PATH = 2
SPMM_NOALLOC_SCRATCH_BYTES = 64 << 20  # SPORDER_SPMM_NOALLOC_SCRATCH_BYTES
SPMM_NOALLOC_TOO_LARGE = 1             # SPORDER_SPMM_NOALLOC_TOO_LARGE
STREAM_READ = 0                        # sporder_stream_op_t
STREAM_WRITE = 1
STREAM_COPY = 2

# Every symbol include/sporder.h declares, with its ctypes signature.
SIGNATURES = {
    "sporder_context_create": ([], vp),
    "sporder_context_destroy": ([vp], None),
    "sporder_hierarchical_matching": (
        [vp, i32, i32, vp, vp, ctypes.c_bool, i32, P(Options), vp, P(HmTiming), P(HmStats)], None),
    "sporder_chunk_greedy": (
        [vp, i32, i32, vp, vp, ctypes.c_bool, i32, f32, i32, vp, P(CgTiming), P(CgStats)], None),
    "sporder_chunk_similarity_greedy": (
        [vp, i32, i32, vp, vp, ctypes.c_bool, i32, f32, i32, vp, P(CsgTiming), P(CsgStats)], None),
    "sporder_reorder": ([vp, i32, i32, vp, vp, vp, vp, i32, vp, vp, vp], None),
    "sporder_count_pillars": ([vp, i32, i32, vp, vp, i32, P(i32)], None),
    "sporder_bench_cusparse_spmm": ([vp, i32, i32, vp, vp, i32, i32, i32, u64, P(f32)], None),
    "sporder_similarity_graph": (
        [vp, i32, i32, vp, vp, ctypes.c_bool, i32, f32, vp, vp, P(SimTiming), P(SimStats)], None),
    "sporder_similarity_graph_exact": (
        [vp, i32, i32, vp, vp, ctypes.c_bool, i32, vp, vp, vp, vp], None),
    "sporder_chunk_similarity_top_k": (
        [vp, i32, i32, vp, vp, ctypes.c_bool, i32, f32, i32, vp, vp], None),
    "sporder_spmm_csr": ([vp, i32, i32, vp, vp, vp, i32, vp, vp, i32, P(f32)], None),
    "sporder_spmm_csr_noalloc": ([vp, i32, i32, vp, vp, vp, i32, vp, vp], i32),
    "sporder_spmm_csr_scaled": ([vp, i32, i32, vp, vp, vp, i32, vp, vp, vp, vp, P(f32)], None),
    "sporder_spmm_plan_create": ([vp, i32, i32, vp, vp, P(SpmmPlanInfo)], vp),
    "sporder_spmm_plan_destroy": ([vp], None),
    "sporder_spmm_csr_plan": ([vp, vp, i32, i32, vp, vp, vp, i32, vp, vp, P(f32)], None),
    "sporder_hbm_stream": ([vp, i32, i32, vp, vp, ctypes.c_int64, i32, P(f32)], None),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load libsporder_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built; run __graft_entry__.build() or "
                "python chunkedgreedy_amd/build.py")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib
