"""Structural reordering-quality metrics on the GPU.

Counterpart of the reference's experiments/quality_metrics.py:36-57 (numpy on
the host) and the pillar count spmatkit.py:1974-1995, for a CSR pattern that
stays in HBM: pillars come from ``sporder.count_pillars`` (the HIP kernel),
the rest from torch operations on the device.  With ``new_order`` the metrics
are those of P A P^T, the pattern after the symmetric reordering.

  pillars   = distinct (row // mu, column) pairs
  tc_blocks = sum over row windows of ceil(pillars_in_window / nu)
  bandwidth = max |i - j|
  profile   = sum over nonempty rows of max(0, i - min column)
  log_gap   = mean over nonzeros of log2(gap + 1), gaps between consecutive
              sorted columns of a row, the first measured from the row index
"""

from __future__ import annotations

MU, NU = 16, 8


def structure_metrics(ptr, ind, new_order=None, *, mu: int = MU, nu: int = NU,
                      ctx=None) -> dict:
    """Metrics of the CSR pattern (ptr, ind), or of P A P^T for a new2old
    permutation `new_order`; all arrays are int32 GPU tensors."""
    import torch

    from chunkedgreedy_amd import sporder

    if new_order is not None:
        ptr, ind = sporder.reorder(ptr, ind, new_order, symmetric=True, ctx=ctx)
    n = ptr.numel() - 1
    nnz = ind.numel()
    dev = ptr.device
    pillars = sporder.count_pillars(ptr, ind, mu, ctx=ctx)
    if nnz == 0:
        return {"pillars": 0, "tc_blocks": 0, "bandwidth": 0, "profile": 0, "log_gap": 0.0}
    deg = (ptr[1:] - ptr[:-1]).long()
    rows = torch.repeat_interleave(torch.arange(n, device=dev), deg)
    cols = ind.long()
    # Columns sorted within each row (the permutation apply sorts; a caller's
    # CSR may not be): sort by (row, column).
    key = rows * n + cols
    key, _ = torch.sort(key)
    rows, cols = key // n, key % n
    win_keys = torch.unique((rows // mu) * n + cols)
    per_win = torch.bincount(win_keys // n)
    tc_blocks = int(((per_win + nu - 1) // nu).sum())
    bandwidth = int((rows - cols).abs().max())
    first = torch.ones(nnz, dtype=torch.bool, device=dev)
    first[1:] = rows[1:] != rows[:-1]
    profile = int(torch.clamp(rows[first] - cols[first], min=0).sum())
    gaps = torch.empty(nnz, dtype=torch.int64, device=dev)
    gaps[1:] = cols[1:] - cols[:-1]
    gaps[first] = (cols[first] - rows[first]).abs()
    log_gap = float(torch.log2(gaps.double() + 1.0).sum() / nnz)
    return {"pillars": pillars, "tc_blocks": tc_blocks, "bandwidth": bandwidth,
            "profile": profile, "log_gap": log_gap, "pillars_check": int(win_keys.numel())}


def reorder_bench_metrics(ptr, ind, new_order=None, *, tc_h: int = 16, tc_w: int = 8,
                          ctx=None) -> dict:
    """The structure columns of the reorder-bench CSV for A or P A P^T
    (spmatkit.py:1704-1717 and 1974-1995, 2037-2060):
      bandwidth    = max over nonzeros of |i - j|
      profile      = sum over nonempty rows of max_j |i - j|
      tc_num       = sum over windows of tc_h rows of ceil(distinct columns / tc_w)
      tc_fill_rate = nnz / (tc_num * tc_h * tc_w)."""
    import torch

    from chunkedgreedy_amd import sporder

    if new_order is not None:
        ptr, ind = sporder.reorder(ptr, ind, new_order, symmetric=True, ctx=ctx)
    n = ptr.numel() - 1
    nnz = ind.numel()
    dev = ptr.device
    out = {"tc_h": tc_h, "tc_w": tc_w}
    if nnz == 0:
        out.update(bandwidth=0, profile=0, tc_num=0, tc_fill_rate=float("nan"))
        return out
    deg = (ptr[1:] - ptr[:-1]).long()
    rows = torch.repeat_interleave(torch.arange(n, device=dev), deg)
    dist = (rows - ind.long()).abs()
    row_max = torch.zeros(n, dtype=torch.int64, device=dev).scatter_reduce(
        0, rows, dist, reduce="amax", include_self=True)
    out["bandwidth"] = int(row_max.max())
    out["profile"] = int(row_max.sum())
    win_keys = torch.unique((rows // tc_h) * n + ind.long())
    per_win = torch.bincount(win_keys // n)
    tc_num = int(((per_win + tc_w - 1) // tc_w).sum())
    out["tc_num"] = tc_num
    out["tc_fill_rate"] = nnz / (tc_num * tc_h * tc_w) if tc_num else float("nan")
    return out
