"""Low-level binding of libsporder_hip.so for torch tensors on a ROCm GPU.

Counterpart of the reference's nanobind extension ``_sporder``
(sporder/python/bindings.cpp:1-582).  Each function keeps that binding's
argument names, validation (ValueError for bad sizes), output allocation and
``(array, timing, stats)`` return shape; outputs are torch tensors on the
input's device.

Inputs are 1-D contiguous torch GPU tensors (or DLPack-capable GPU arrays,
converted with ``torch.from_dlpack``).  Before each call the caller's current
torch stream is synchronized, because the library runs on its own stream
(the reference leaves that to the caller, sporder/include/sporder.h:22-25).
ctypes releases the GIL for the duration of the foreign call, as the
reference binding does (bindings.cpp:338-345).
"""

from __future__ import annotations

import ctypes

import torch

from .. import _lib

INT32_MAX = 2**31 - 1


class Context:
    """A library context (private HIP stream + workspace) bound to the device
    current at creation (reference bindings.cpp:23-38)."""

    def __init__(self):
        _require_gpu()
        self._lib = _lib.load()
        self.device = torch.cuda.current_device()
        self.handle = self._lib.sporder_context_create()
        if not self.handle:
            raise RuntimeError("sporder_context_create failed")

    def close(self):
        if getattr(self, "handle", None):
            with torch.cuda.device(self.device):
                self._lib.sporder_context_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_default_ctx = None


def default_context() -> Context:
    """Process-lifetime shared context, created on first use
    (reference bindings.cpp:40-43)."""
    global _default_ctx
    if _default_ctx is None:
        _default_ctx = Context()
    return _default_ctx


def _require_gpu():
    if not torch.cuda.is_available():
        raise RuntimeError("sporder needs a ROCm GPU; torch.cuda.is_available() is False")


def _as_tensor(a, name):
    if isinstance(a, torch.Tensor):
        return a
    if hasattr(a, "__dlpack__"):
        return torch.from_dlpack(a)
    raise TypeError(f"{name} must be a torch tensor or a DLPack-capable GPU array")


def _gpu_in(a, dtype, name):
    """1-D, C-contiguous GPU tensor of `dtype` (reference gpu_in, bindings.cpp:17-19)."""
    t = _as_tensor(a, name)
    if not t.is_cuda:
        raise TypeError(f"{name} must be a GPU tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must have dtype {dtype}, got {t.dtype}")
    if t.dim() != 1:
        raise TypeError(f"{name} must be 1-D")
    if not t.is_contiguous():
        raise TypeError(f"{name} must be contiguous")
    return t


def _resolve(ctx, ref):
    c = ctx if ctx is not None else default_context()
    if ref.device.index != c.device:
        raise ValueError(f"arrays live on cuda:{ref.device.index} but the context is on "
                         f"cuda:{c.device}")
    torch.cuda.current_stream(ref.device).synchronize()
    return c


def _sizes(ptr, ind):
    if ptr.numel() < 2:
        raise ValueError("ptr must have length n+1 (at least 2)")
    n = ptr.numel() - 1
    nnz = ind.numel()
    if n > INT32_MAX or nnz > INT32_MAX:
        raise ValueError("matrix too large for int32 indexing")
    return n, nnz


def _addr(t):
    return ctypes.c_void_p(t.data_ptr())


def chunk_similarity_greedy(ptr, ind, is_symmetric=False, k=0, oversampling=0.0,
                            chunk_size=0, with_timing=False, with_stats=False,
                            ctx=None):
    """Reference bindings.cpp:317-374."""
    ptr = _gpu_in(ptr, torch.int32, "ptr")
    ind = _gpu_in(ind, torch.int32, "ind")
    n, nnz = _sizes(ptr, ind)
    c = _resolve(ctx, ptr)
    new_order = torch.empty(n, dtype=torch.int32, device=ptr.device)
    timing = _lib.CsgTiming()
    stats = _lib.CsgStats()
    c._lib.sporder_chunk_similarity_greedy(
        c.handle, n, nnz, _addr(ptr), _addr(ind), bool(is_symmetric), int(k),
        float(oversampling), int(chunk_size), _addr(new_order),
        ctypes.byref(timing) if with_timing else None,
        ctypes.byref(stats) if with_stats else None)
    timing_info = None
    if with_timing:
        timing_info = {"wall_ms": timing.wall_ms, "csr2csc_ms": timing.csr2csc_ms,
                       "similarity_ms": timing.similarity_ms,
                       "chunk_greedy_ms": timing.chunk_greedy_ms}
    stats_info = None
    if with_stats:
        stats_info = {"k_used": stats.k_used, "m_used": stats.m_used,
                      "avg_degree": stats.avg_degree,
                      "avg_edge_weight": stats.avg_edge_weight,
                      "zero_degree_rows": stats.zero_degree_rows,
                      "chunk_size_used": stats.chunk_size_used,
                      "chain_restarts": stats.chain_restarts,
                      "avg_followed_weight": stats.avg_followed_weight}
    return new_order, timing_info, stats_info


def chunk_greedy(ptr, ind, is_symmetric=False, k=0, oversampling=0.0, chunk_size=0,
                 with_timing=False, with_stats=False, ctx=None):
    """Reference bindings.cpp:258-312."""
    ptr = _gpu_in(ptr, torch.int32, "ptr")
    ind = _gpu_in(ind, torch.int32, "ind")
    n, nnz = _sizes(ptr, ind)
    c = _resolve(ctx, ptr)
    new_order = torch.empty(n, dtype=torch.int32, device=ptr.device)
    timing = _lib.CgTiming()
    stats = _lib.CgStats()
    c._lib.sporder_chunk_greedy(
        c.handle, n, nnz, _addr(ptr), _addr(ind), bool(is_symmetric), int(k),
        float(oversampling), int(chunk_size), _addr(new_order),
        ctypes.byref(timing) if with_timing else None,
        ctypes.byref(stats) if with_stats else None)
    timing_info = None
    if with_timing:
        timing_info = {"wall_ms": timing.wall_ms, "csr2csc_ms": timing.csr2csc_ms,
                       "similarity_ms": timing.similarity_ms,
                       "chunk_greedy_ms": timing.chunk_greedy_ms}
    stats_info = None
    if with_stats:
        stats_info = {"k_used": stats.k_used, "m_used": stats.m_used,
                      "avg_degree": stats.avg_degree,
                      "avg_edge_weight": stats.avg_edge_weight,
                      "zero_degree_rows": stats.zero_degree_rows,
                      "chunk_size_used": stats.chunk_size_used,
                      "chain_restarts": stats.chain_restarts,
                      "avg_followed_weight": stats.avg_followed_weight,
                      "cut_weight_fraction": stats.cut_weight_fraction}
    return new_order, timing_info, stats_info


def count_pillars(ptr, ind, height, ctx=None):
    """Reference bindings.cpp:204-227."""
    ptr = _gpu_in(ptr, torch.int32, "ptr")
    ind = _gpu_in(ind, torch.int32, "ind")
    if ptr.numel() < 2:
        raise ValueError("ptr must have length n+1 (at least 2)")
    if int(height) < 1:
        raise ValueError("height must be >= 1")
    n, nnz = _sizes(ptr, ind)
    c = _resolve(ctx, ptr)
    count = ctypes.c_int32()
    c._lib.sporder_count_pillars(c.handle, n, nnz, _addr(ptr), _addr(ind), int(height),
                                 ctypes.byref(count))
    return int(count.value)


def reorder(ptr, ind, val=None, new_order=None, symmetric=False, ctx=None):
    """Reference bindings.cpp:151-202."""
    ptr = _gpu_in(ptr, torch.int32, "ptr")
    ind = _gpu_in(ind, torch.int32, "ind")
    if new_order is None:
        raise TypeError("new_order is required")
    new_order = _gpu_in(new_order, torch.int32, "new_order")
    if ptr.numel() < 2:
        raise ValueError("ptr must have length n+1 (at least 2)")
    n = ptr.numel() - 1
    nnz = ind.numel()
    if new_order.numel() != n:
        raise ValueError("new_order must have length n")
    if n > INT32_MAX or nnz > INT32_MAX:
        raise ValueError("matrix too large for int32 indexing")
    val_in = None
    if val is not None:
        val_in = _gpu_in(val, torch.float32, "val")
        if val_in.device != ptr.device:
            raise ValueError("val must live on the same device as ptr")
    c = _resolve(ctx, ptr)
    ptr_new = torch.empty(n + 1, dtype=torch.int32, device=ptr.device)
    ind_new = torch.empty(max(nnz, 1), dtype=torch.int32, device=ptr.device)
    val_new = None
    if val_in is not None:
        val_new = torch.empty(max(nnz, 1), dtype=torch.float32, device=ptr.device)
    c._lib.sporder_reorder(
        c.handle, n, nnz, _addr(ptr), _addr(ind),
        _addr(val_in) if val_in is not None else None, _addr(new_order),
        _lib.REORDER_SYMMETRIC if symmetric else _lib.REORDER_ROWS, _addr(ptr_new),
        _addr(ind_new), _addr(val_new) if val_new is not None else None)
    if val_new is None:
        return ptr_new, ind_new[:nnz]
    return ptr_new, ind_new[:nnz], val_new[:nnz]


def bench_cusparse_spmm(ptr, ind, cols, warmup=3, repeat=10, seed=0, ctx=None):
    """Reference bindings.cpp:229-256 (the timed kernel is this library's SpMM)."""
    ptr = _gpu_in(ptr, torch.int32, "ptr")
    ind = _gpu_in(ind, torch.int32, "ind")
    if ptr.numel() < 2:
        raise ValueError("ptr must have length n+1 (at least 2)")
    if warmup < 0 or repeat < 0:
        raise ValueError("warmup and repeat must be >= 0")
    if cols < 1:
        raise ValueError("cols must be >= 1")
    n, nnz = _sizes(ptr, ind)
    c = _resolve(ctx, ptr)
    out = ctypes.c_float(0.0)
    c._lib.sporder_bench_cusparse_spmm(c.handle, n, nnz, _addr(ptr), _addr(ind), int(cols),
                                       int(warmup), int(repeat), int(seed) & (2**64 - 1),
                                       ctypes.byref(out))
    return out.value


def similarity_graph(ptr, ind, is_symmetric=False, k=0, oversampling=0.0,
                     with_timing=False, with_stats=False, ctx=None):
    """Reference bindings.cpp:376-430 (global sketch)."""
    ptr = _gpu_in(ptr, torch.int32, "ptr")
    ind = _gpu_in(ind, torch.int32, "ind")
    n, nnz = _sizes(ptr, ind)
    c = _resolve(ctx, ptr)
    k_used = int(k) if k > 0 else min(32, max(16, 2 * (nnz // n)))
    idx = torch.empty(n * k_used, dtype=torch.int32, device=ptr.device)
    wgt = torch.empty(n * k_used, dtype=torch.float32, device=ptr.device)
    timing = _lib.SimTiming()
    stats = _lib.SimStats()
    c._lib.sporder_similarity_graph(
        c.handle, n, nnz, _addr(ptr), _addr(ind), bool(is_symmetric), int(k),
        float(oversampling), _addr(idx), _addr(wgt),
        ctypes.byref(timing) if with_timing else None,
        ctypes.byref(stats) if with_stats else None)
    timing_info = None
    if with_timing:
        timing_info = {"wall_ms": timing.wall_ms, "csr2csc_ms": timing.csr2csc_ms,
                       "similarity_ms": timing.similarity_ms, "unpack_ms": timing.unpack_ms}
    stats_info = None
    if with_stats:
        stats_info = {"k_used": stats.k_used, "m_used": stats.m_used,
                      "avg_degree": stats.avg_degree,
                      "avg_edge_weight": stats.avg_edge_weight,
                      "zero_degree_rows": stats.zero_degree_rows}
    return idx, wgt, timing_info, stats_info


def chunk_similarity_top_k(ptr, ind, k, oversampling, chunk_size, is_symmetric=False,
                           ctx=None):
    """The csg sketch table (new export, no reference binding): (indices, weights)
    as n x k tensors."""
    ptr = _gpu_in(ptr, torch.int32, "ptr")
    ind = _gpu_in(ind, torch.int32, "ind")
    n, nnz = _sizes(ptr, ind)
    if k <= 0 or oversampling < 1.0 or chunk_size < 1:
        raise ValueError("k, oversampling and chunk_size must be resolved (k > 0, "
                         "oversampling >= 1, chunk_size >= 1)")
    if int(k * oversampling) > 512:
        raise ValueError("k * oversampling must be <= 512")
    c = _resolve(ctx, ptr)
    idx = torch.empty(n * k, dtype=torch.int32, device=ptr.device)
    wgt = torch.empty(n * k, dtype=torch.float32, device=ptr.device)
    c._lib.sporder_chunk_similarity_top_k(c.handle, n, nnz, _addr(ptr), _addr(ind),
                                          bool(is_symmetric), int(k), float(oversampling),
                                          int(chunk_size), _addr(idx), _addr(wgt))
    return idx.view(n, k), wgt.view(n, k)


class SpmmPlan:
    """An SpMM plan of one CSR pattern (new export): the blocked tiles, whose
    8-row blocks load each distinct column's B row once, and their (column,
    row mask) entries.  Owns device memory on the context's device until
    closed or collected."""

    def __init__(self, ptr, ind, ctx=None):
        ptr = _gpu_in(ptr, torch.int32, "ptr")
        ind = _gpu_in(ind, torch.int32, "ind")
        self.n, self.nnz = _sizes(ptr, ind)
        self._ctx = _resolve(ctx, ptr)
        self._lib = self._ctx._lib
        self.device = ptr.device
        info = _lib.SpmmPlanInfo()
        self.handle = self._lib.sporder_spmm_plan_create(self._ctx.handle, self.n, self.nnz,
                                                         _addr(ptr), _addr(ind),
                                                         ctypes.byref(info))
        if not self.handle:
            raise RuntimeError("sporder_spmm_plan_create failed")
        self.info = {name: getattr(info, name) for name, _ in _lib.SpmmPlanInfo._fields_}

    def close(self):
        if getattr(self, "handle", None):
            self._lib.sporder_spmm_plan_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def spmm_plan(ptr, ind, ctx=None):
    return SpmmPlan(ptr, ind, ctx=ctx)


def spmm_csr(ptr, ind, val, B, out=None, algo="row_split", ctx=None, plan=None):
    """C = A @ B for CSR A and row-major dense B (new export).  Returns
    (C, kernel_ms).  With a plan of this pattern, the planned SpMM (same
    result as algo "row_split")."""
    ptr = _gpu_in(ptr, torch.int32, "ptr")
    ind = _gpu_in(ind, torch.int32, "ind")
    val = _gpu_in(val, torch.float32, "val")
    n, nnz = _sizes(ptr, ind)
    if val.numel() != nnz:
        raise ValueError("val must have length nnz")
    B = _as_tensor(B, "B")
    if not B.is_cuda or B.dtype != torch.float32 or B.dim() != 2 or B.shape[0] != n:
        raise ValueError("B must be an (n, N) float32 GPU tensor")
    B = B.contiguous()
    cols = B.shape[1]
    if cols < 1:
        raise ValueError("B must have at least one column")
    if out is None:
        out = torch.empty((n, cols), dtype=torch.float32, device=B.device)
    elif out.shape != (n, cols) or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError("out must be a contiguous (n, N) float32 tensor")
    codes = {"auto": _lib.SPMM_AUTO, "row_split": _lib.SPMM_ROW_SPLIT,
             "merge_path": _lib.SPMM_MERGE_PATH}
    if algo not in codes:
        raise ValueError(f"algo must be one of {sorted(codes)}")
    c = _resolve(ctx, ptr)
    ms = ctypes.c_float(0.0)
    if plan is not None:
        if algo == "merge_path":
            raise ValueError("a plan runs the row-split order; algo must be auto or row_split")
        if not plan.handle or plan.n != n or plan.nnz != nnz or plan.device != ptr.device:
            raise ValueError("plan was made for another matrix or device")
        c._lib.sporder_spmm_csr_plan(c.handle, plan.handle, n, nnz, _addr(ptr), _addr(ind),
                                     _addr(val), cols, _addr(B), _addr(out), ctypes.byref(ms))
        return out, ms.value
    c._lib.sporder_spmm_csr(c.handle, n, nnz, _addr(ptr), _addr(ind), _addr(val), cols,
                            _addr(B), _addr(out), codes[algo], ctypes.byref(ms))
    return out, ms.value


def spmm_csr_scaled(ptr, ind, val, B, row_scale=None, col_scale=None, nz_col_scale=None,
                    out=None, ctx=None):
    """C = diag(row_scale) A diag(col_scale) B with the row-split kernels (new
    export).  Bit-identical to (row_scale[:, None] * spmm_csr(A,
    col_scale[:, None] * B)); either scale may be None.  The kernels take the
    column scales per nonzero (col_scale[ind]): pass them as nz_col_scale to
    skip that gather when the pattern is reused.  Returns (C, kernel_ms)."""
    ptr = _gpu_in(ptr, torch.int32, "ptr")
    ind = _gpu_in(ind, torch.int32, "ind")
    val = _gpu_in(val, torch.float32, "val")
    n, nnz = _sizes(ptr, ind)
    if val.numel() != nnz:
        raise ValueError("val must have length nnz")
    B = _as_tensor(B, "B")
    if not B.is_cuda or B.dtype != torch.float32 or B.dim() != 2 or B.shape[0] != n:
        raise ValueError("B must be an (n, N) float32 GPU tensor")
    B = B.contiguous()
    cols = B.shape[1]
    if cols < 1:
        raise ValueError("B must have at least one column")

    def checked(name, sc, length):
        sc = _as_tensor(sc, name)
        if not sc.is_cuda or sc.dtype != torch.float32 or sc.numel() != length \
                or sc.device != B.device:
            raise ValueError(f"{name} must be {length} float32 values on B's device")
        return sc.reshape(length).contiguous()

    rs = None if row_scale is None else checked("row_scale", row_scale, n)
    if nz_col_scale is not None:
        if col_scale is not None:
            raise ValueError("give col_scale or nz_col_scale, not both")
        nz = checked("nz_col_scale", nz_col_scale, nnz)
    elif col_scale is not None:
        nz = checked("col_scale", col_scale, n)[ind.long()] if nnz else \
            torch.empty(0, dtype=torch.float32, device=B.device)
    else:
        nz = None
    if out is None:
        out = torch.empty((n, cols), dtype=torch.float32, device=B.device)
    elif out.shape != (n, cols) or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError("out must be a contiguous (n, N) float32 tensor")
    c = _resolve(ctx, ptr)
    ms = ctypes.c_float(0.0)
    c._lib.sporder_spmm_csr_scaled(c.handle, n, nnz, _addr(ptr), _addr(ind), _addr(val), cols,
                                   _addr(B), _addr(rs) if rs is not None else None,
                                   _addr(nz) if nz is not None and nz.numel() else None,
                                   _addr(out), ctypes.byref(ms))
    return out, ms.value


def spmm_csr_noalloc(ptr, ind, val, B, out, ctx=None):
    """C = A @ B into the caller's `out` with no device allocation by the
    library (new export, the row-split in the stated order).  Raises
    ValueError when the matrix's long rows need more scratch than the
    library's static array holds."""
    ptr = _gpu_in(ptr, torch.int32, "ptr")
    ind = _gpu_in(ind, torch.int32, "ind")
    val = _gpu_in(val, torch.float32, "val")
    n, nnz = _sizes(ptr, ind)
    if val.numel() != nnz:
        raise ValueError("val must have length nnz")
    B = _as_tensor(B, "B")
    if not B.is_cuda or B.dtype != torch.float32 or B.dim() != 2 or B.shape[0] != n \
            or not B.is_contiguous():
        raise ValueError("B must be a contiguous (n, N) float32 GPU tensor")
    cols = B.shape[1]
    if cols < 1:
        raise ValueError("B must have at least one column")
    if (out is None or out.shape != (n, cols) or out.dtype != torch.float32
            or not out.is_contiguous() or out.device != B.device):
        raise ValueError("out must be a contiguous (n, N) float32 tensor on B's device")
    c = _resolve(ctx, ptr)
    rc = c._lib.sporder_spmm_csr_noalloc(c.handle, n, nnz, _addr(ptr), _addr(ind), _addr(val),
                                         cols, _addr(B), _addr(out))
    if rc == _lib.SPMM_NOALLOC_TOO_LARGE:
        raise ValueError(
            f"the long rows of this matrix need more than the "
            f"{_lib.SPMM_NOALLOC_SCRATCH_BYTES >> 20} MiB no-allocation scratch at N={cols}; "
            "use spmm_csr")
    if rc != 0:
        raise RuntimeError(f"sporder_spmm_csr_noalloc returned {rc}")
    return out


def _not_built(name):
    def fn(*args, **kwargs):
        raise NotImplementedError(f"sporder.{name} is not part of this build")

    fn.__name__ = name
    return fn


# Entry points the reference imports at package load (reference
# sporder/python/sporder/__init__.py:3-13) that this build does not provide.
hierarchical_matching = _not_built("hierarchical_matching")
similarity_graph_exact = _not_built("similarity_graph_exact")
