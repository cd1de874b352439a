"""Counterparts of the reference bench plugins that call the hot path.

* Reorder plugins for ``sporder-csg`` and ``sporder-cg``:
  ``reorder(csr, params)`` / ``reorder_cg(csr, params) -> ReorderResult``
  (reference bench/reorder/reorder_bench/methods/sporder_csg.py:25-70 and
  sporder_cg.py:25-70; ``REORDER_METHODS`` maps the method names), with
  ``prep_sporder_gpu`` (loader.py:63-93), ``flush_l2`` (timing.py:29-42),
  ``row_perm_from_order`` (loader.py:124-128), ``timed_ms`` (timing.py:8-15)
  and the ``ReorderResult`` record (types.py:9-17).  Device arrays are torch
  tensors instead of CuPy arrays.
* SpMM plugin: the ``SpMMMethod`` interface (bench/spmm/spmm_bench/base.py:8-87)
  and a ``hip-csr-spmm`` method backed by ``sporder.spmm_csr``, with
  ``generate_dense`` (utils.py:219-225) and the warmup/iteration timing loop
  (batch_bench.py:516-529).

``flush_l2`` writes 1 GiB (the reference writes 2x the L2 size): on MI355X
that covers the per-XCD L2s and the 256 MB Infinity Cache.
"""

from __future__ import annotations

import time
from abc import ABC, abstractmethod
from contextlib import contextmanager
from dataclasses import dataclass, field
from typing import Any, Iterator

import numpy as np
import scipy.sparse

INT32_MAX = np.iinfo(np.int32).max


@dataclass
class ReorderResult:
    """Reference bench/reorder/reorder_bench/types.py:9-17."""

    row_perm: np.ndarray
    reorder_time_ms: float
    prep_time_ms: float = 0.0
    perm_trans_ms: float = 0.0
    timing_breakdown: dict[str, float] = field(default_factory=dict)
    effective_params: dict[str, Any] = field(default_factory=dict)
    env_extra: dict[str, Any] = field(default_factory=dict)


@contextmanager
def timed_ms() -> Iterator[list[float]]:
    bucket = [0.0]
    t0 = time.perf_counter()
    try:
        yield bucket
    finally:
        bucket[0] = (time.perf_counter() - t0) * 1000.0


def flush_l2(device: int | str = 0, nbytes: int = 1 << 30) -> None:
    """Evict the GPU caches by writing `nbytes` (default 1 GiB)."""
    import torch

    dev = torch.device(device if isinstance(device, str) else f"cuda:{device}")
    buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    buf.zero_()
    torch.cuda.synchronize(dev)
    del buf


def prep_sporder_gpu(csr: scipy.sparse.csr_matrix, *, detect_symmetric: bool = True,
                     device: str = "cuda:0"):
    """Sort the CSR, detect pattern symmetry, upload int32 ptr/ind.

    Returns (ptr, ind, is_symmetric, prep_ms).  Symmetry is tested as the
    reference does, ``(A != A.T).nnz == 0`` on the matrix as given.
    """
    import torch

    nrows = int(csr.shape[0])
    nnz = int(csr.nnz)
    if nrows > INT32_MAX or nnz > INT32_MAX:
        raise ValueError(f"sporder requires n and nnz within int32; got n={nrows}, nnz={nnz}")
    with timed_ms() as bucket:
        out = csr.copy()
        out.sort_indices()
        is_symmetric = bool((out != out.T).nnz == 0) if detect_symmetric else False
        ptr = torch.from_numpy(np.ascontiguousarray(out.indptr, dtype=np.int32)).to(device)
        ind = torch.from_numpy(np.ascontiguousarray(out.indices, dtype=np.int32)).to(device)
        torch.cuda.synchronize(device)
    return ptr, ind, is_symmetric, bucket[0]


def row_perm_from_order(order, nrows: int) -> np.ndarray:
    perm = np.asarray(order, dtype=np.int64)
    if perm.shape[0] != nrows:
        raise ValueError(f"perm length {perm.shape[0]} != nrows {nrows}")
    return perm


def _reorder_with(entry, csr: scipy.sparse.csr_matrix, params: dict[str, Any]) -> ReorderResult:
    """Warmup call, cache flush, timed call; reorder_time_ms is the library's
    wall_ms (reference sporder_csg.py:25-70 and sporder_cg.py:25-70 share this
    shape)."""
    auto_detect = bool(params.get("auto_detect_symmetric", True))
    ptr, ind, is_symmetric, prep_ms = prep_sporder_gpu(csr, detect_symmetric=auto_detect)
    nrows = csr.shape[0]
    call_kwargs = {
        "is_symmetric": is_symmetric,
        "k": int(params.get("k", 0)),
        "oversampling": float(params.get("oversampling", 0.0)),
        "chunk_size": int(params.get("chunk_size", 0)),
        "with_stats": False,
    }
    entry(ptr, ind, with_timing=False, **call_kwargs)
    flush_l2(ptr.device.index or 0)
    order, timing = entry(ptr, ind, with_timing=True, **call_kwargs)
    breakdown = {
        "csr2csc_ms": float(timing.get("csr2csc_ms", 0.0)),
        "similarity_ms": float(timing.get("similarity_ms", 0.0)),
        "chunk_greedy_ms": float(timing.get("chunk_greedy_ms", 0.0)),
    }
    with timed_ms() as bucket:
        row_perm = row_perm_from_order(order.cpu().numpy().astype(np.int64), nrows)
    return ReorderResult(row_perm=row_perm, reorder_time_ms=float(timing["wall_ms"]),
                         prep_time_ms=prep_ms, perm_trans_ms=bucket[0],
                         timing_breakdown=breakdown,
                         effective_params={"is_symmetric": is_symmetric})


def reorder(csr: scipy.sparse.csr_matrix, params: dict[str, Any]) -> ReorderResult:
    """The ``sporder-csg`` reorder method (reference sporder_csg.py:25-70)."""
    from chunkedgreedy_amd import sporder

    return _reorder_with(sporder.chunk_similarity_greedy, csr, params)


def reorder_cg(csr: scipy.sparse.csr_matrix, params: dict[str, Any]) -> ReorderResult:
    """The ``sporder-cg`` reorder method, "CG w/o Stage 1" (reference
    sporder_cg.py:25-70)."""
    from chunkedgreedy_amd import sporder

    return _reorder_with(sporder.chunk_greedy, csr, params)


REORDER_METHODS = {"sporder-csg": reorder, "sporder-cg": reorder_cg}


def apply_row_perm(csr: scipy.sparse.csr_matrix, row_perm) -> scipy.sparse.csr_matrix:
    """P A P^T on the host (reference spmatkit/spmatkit.py:963-982)."""
    if not scipy.sparse.isspmatrix_csr(csr):
        csr = csr.tocsr()
    n, m = csr.shape
    if n != m:
        raise ValueError(f"reorder perm requires a square matrix, got shape {csr.shape}")
    perm = np.asarray(row_perm, dtype=np.int64)
    if perm.shape[0] != n:
        raise ValueError(f"row_perm length {perm.shape[0]} != matrix dimension {n}")
    return csr[perm, :][:, perm].tocsr()


# ---- SpMM plugin ------------------------------------------------------------


class SpMMMethod(ABC):
    """Interface of the reference SpMM wrappers (bench/spmm/spmm_bench/base.py:8-87)."""

    @property
    @abstractmethod
    def name(self) -> str: ...

    @property
    def uses_feature_dim(self) -> bool:
        return True

    @property
    def uses_cuda(self) -> bool:
        return True

    @property
    @abstractmethod
    def tc_h(self) -> int: ...

    @property
    @abstractmethod
    def tc_w(self) -> int: ...

    @abstractmethod
    def build(self) -> None: ...

    @abstractmethod
    def prepare(self, A_csr: Any) -> Any: ...

    @abstractmethod
    def run(self, prepared_A: Any, B) -> tuple[Any, float]: ...

    @classmethod
    def create(cls, name: str) -> "SpMMMethod":
        registry = {"hip-csr-spmm": HipCsrSpMM, "hip-csr-spmm-merge": HipCsrSpMMMerge}
        if name not in registry:
            raise ValueError(f"Unknown method: {name}. Available: {list(registry)}")
        return registry[name]()


class HipCsrSpMM(SpMMMethod):
    """CSR SpMM in the library's stated row-split order.  prepare (untimed in
    the harness) uploads the CSR and builds an SpMM plan, so tiles of rows
    that share columns run in 8-row blocks; run is one planned SpMM."""

    algo = "row_split"
    planned = True

    @property
    def name(self) -> str:
        return "hip-csr-spmm"

    @property
    def tc_h(self) -> int:
        return 0

    @property
    def tc_w(self) -> int:
        return 0

    def build(self) -> None:
        from chunkedgreedy_amd import _lib

        _lib.load()

    def prepare(self, A_csr: scipy.sparse.csr_matrix):
        import torch

        n, m = A_csr.shape
        if n != m:
            raise RuntimeError(f"{self.name} requires a square CSR matrix; got {n}x{m}")
        a = A_csr.tocsr()
        a.sort_indices()
        from chunkedgreedy_amd import sporder

        dev = torch.device("cuda:0")
        ptr = torch.from_numpy(np.ascontiguousarray(a.indptr, np.int32)).to(dev)
        ind = torch.from_numpy(np.ascontiguousarray(a.indices, np.int32)).to(dev)
        val = torch.from_numpy(np.ascontiguousarray(a.data, np.float32)).to(dev)
        plan = sporder.spmm_plan(ptr, ind) if self.planned else None
        return ptr, ind, val, plan

    def run(self, prepared_A, B):
        import torch

        from chunkedgreedy_amd import sporder

        ptr, ind, val, plan = prepared_A
        out = torch.empty((B.size(0), B.size(1)), dtype=torch.float32, device=B.device)
        out, ms = sporder.spmm_csr(ptr, ind, val, B.contiguous(), out=out, algo=self.algo,
                                   plan=plan)
        return out, float(ms)


class HipCsrSpMMMerge(HipCsrSpMM):
    """Merge-path variant (balanced nonzeros per wave, for skewed rows)."""

    algo = "merge_path"
    planned = False

    @property
    def name(self) -> str:
        return "hip-csr-spmm-merge"


def generate_dense(num_nodes: int, feature_dim: int, device: str = "cuda", seed: int = 42,
                   dtype=None):
    """Reference bench/spmm/spmm_bench/utils.py:219-225."""
    import torch

    gen = torch.Generator(device=device).manual_seed(seed)
    return torch.randn((num_nodes, feature_dim), generator=gen,
                       dtype=dtype or torch.float32, device=device)


def time_run(method: SpMMMethod, prepared, B, warmup: int = 30, iterations: int = 100) -> float:
    """Mean per-launch kernel ms (reference batch_bench.py:516-529)."""
    for _ in range(warmup):
        method.run(prepared, B)
    total = 0.0
    for _ in range(iterations):
        _, ms = method.run(prepared, B)
        total += ms
    return total / iterations
