"""Measure the path on the five synthetic configurations (one GPU).

For each configuration: the csg reorder (``chunk_similarity_greedy``, warmup,
then a 1 GiB cache flush before each timed call, median wall of ``--repeats``
calls with its stage spans and stats), the permutation apply P A P^T with
values, and the CSR SpMM on the original and on the reordered matrix at the
configuration's widths (warmup 5, median of 20 launch times, B = randn seed
42, the same B for both matrices).  Prints one JSON record per configuration.

Algorithmic bytes of an SpMM launch: 4(n+1) + 8 nnz + 8 n N (A once, B once,
C once).

With ``--candidates`` (host only, no GPU): per configuration, how many rows'
chunk-restricted candidate streams hold at most M distinct items (the
space-saving sketch never evicts there) and how much of the stream work those
rows hold, plus the longest streams' distinct counts (``candidate_stats``).

With ``--runs`` (host only): the rows the permutation apply sends to its
long-row stage and their runs of equal column block (``run_stats``).

Configurations: C1..C5 (synth.CONFIGS) and the inputs with in-chunk locality
C2r, C4n, RGG20, C5d (synth.LOCALITY).

Usage:  python -m chunkedgreedy_amd.sweep [--cfg C1,C2,C3,C4,C5] [--no-spmm]
        [--algos row_split,merge_path,plan] [--cg] [--candidates] [--runs]
        [--widths 32,256] [--spmm-iters K] [--spmm-warmup W] [--calibrate BYTES]
        [--cache DIR]
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys
import time

import numpy as np

WIDTHS = {"C1": [32], "C2": [32, 128], "C3": [32, 64, 256], "C4": [16, 32, 64, 128, 256],
          "C5": [128],
          # inputs with in-chunk locality (synth.LOCALITY)
          "C2r": [128], "C4n": [32], "RGG20": [32, 128], "C5d": [128]}


def generators() -> dict:
    from chunkedgreedy_amd import synth

    return {**synth.CONFIGS, **synth.LOCALITY}


def generate(name: str, cache: str | None = None):
    """The configuration's CSR (ptr, ind, val), from `cache`/<name>.npz when
    present, else generated (and written there when `cache` is given), so
    that several runs of one session generate each input once."""
    import os

    path = os.path.join(cache, f"{name}.npz") if cache else None
    if path and os.path.exists(path):
        with np.load(path) as z:
            return z["ptr"], z["ind"], z["val"]
    ptr, ind, val = generators()[name]()
    if path:
        os.makedirs(cache, exist_ok=True)
        np.savez(path, ptr=ptr, ind=ind, val=val)
    return ptr, ind, val


def spmm_bytes(n: int, nnz: int, N: int) -> int:
    return 4 * (n + 1) + 8 * nnz + 8 * n * N


def _spmm_ms(sporder, ctx, ptr, ind, val, B, algo, iters=20, warmup=5):
    """Median launch time; algo "plan" times the planned SpMM, the plan made
    beforehand and untimed (the harness's prepare step)."""
    import torch

    plan = sporder.spmm_plan(ptr, ind, ctx=ctx) if algo == "plan" else None
    kw = {"plan": plan} if plan is not None else {"algo": algo}
    out = torch.empty(B.shape, dtype=torch.float32, device=B.device)
    for _ in range(warmup):
        sporder.spmm_csr(ptr, ind, val, B, out=out, ctx=ctx, **kw)
    ms = statistics.median(
        sporder.spmm_csr(ptr, ind, val, B, out=out, ctx=ctx, **kw)[1] for _ in range(iters))
    if plan is not None:
        plan.close()
    return ms


def calibration_copy(nbytes: int, ctx) -> None:
    """One launch of the library's copy kernel over nbytes (reads nbytes,
    writes nbytes): the reference dispatch by which a `rocprofv3 --pmc` run
    scales FETCH_SIZE and WRITE_SIZE to bytes."""
    import ctypes

    import torch

    from chunkedgreedy_amd import _lib

    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    ms = ctypes.c_float()
    _lib.load().sporder_hbm_stream(ctx.handle, _lib.STREAM_COPY, 0, dst.data_ptr(),
                                   src.data_ptr(), nbytes, 1, ctypes.byref(ms))
    del src, dst
    print(f"[calibration] sporder_hbm_stream copy of {nbytes} bytes: {ms.value:.4f} ms",
          file=sys.stderr, flush=True)


def measure(name: str, *, spmm=True, algos=("row_split",), repeats=3, cg=False,
            widths=None, spmm_iters=20, spmm_warmup=5, calibrate=0, cache=None) -> dict:
    import torch

    from chunkedgreedy_amd import sporder, synth

    gens = generators()
    dev = torch.device("cuda:0")
    ctx = sporder.Context()
    if calibrate > 0:
        calibration_copy(calibrate, ctx)
    t0 = time.time()
    ptr_h, ind_h, val_h = generate(name, cache)
    n, nnz = ptr_h.shape[0] - 1, ind_h.shape[0]
    sym = synth.is_pattern_symmetric(ptr_h, ind_h)
    print(f"[{name}] generated n={n} nnz={nnz} symmetric={sym} in {time.time() - t0:.1f}s",
          file=sys.stderr, flush=True)
    ptr, ind, val = (torch.from_numpy(a).to(dev) for a in (ptr_h, ind_h, val_h))
    rec = {"config": name, "n": n, "nnz": nnz, "symmetric": sym,
           "max_row": int(np.diff(ptr_h).max())}

    sporder.chunk_similarity_greedy(ptr, ind, is_symmetric=sym, ctx=ctx)  # warmup
    flush = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    runs = []
    for _ in range(repeats):
        flush.zero_()
        torch.cuda.synchronize()
        order, timing = sporder.chunk_similarity_greedy(ptr, ind, is_symmetric=sym,
                                                        with_timing=True, ctx=ctx)
        runs.append(timing)
    runs.sort(key=lambda t: t["wall_ms"])
    rec["csg"] = runs[len(runs) // 2]
    _, stats = sporder.chunk_similarity_greedy(ptr, ind, is_symmetric=sym, with_stats=True,
                                               ctx=ctx)
    rec["csg_stats"] = stats
    print(f"[{name}] csg {rec['csg']}", file=sys.stderr, flush=True)
    if cg:
        flush.zero_()
        torch.cuda.synchronize()
        _, timing = sporder.chunk_greedy(ptr, ind, is_symmetric=sym, with_timing=True, ctx=ctx)
        rec["cg"] = timing
        print(f"[{name}] cg {timing}", file=sys.stderr, flush=True)
    del flush

    sporder.reorder(ptr, ind, order, val=val, symmetric=True, ctx=ctx)  # warmup
    perm_ms = []
    for _ in range(5):
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        p2, i2, v2 = sporder.reorder(ptr, ind, order, val=val, symmetric=True, ctx=ctx)
        torch.cuda.synchronize()
        perm_ms.append((time.perf_counter() - t1) * 1e3)
    rec["permute_ms"] = statistics.median(perm_ms)
    print(f"[{name}] permutation apply {rec['permute_ms']:.3f} ms (median of 5)",
          file=sys.stderr, flush=True)

    if spmm:
        if "plan" in algos:
            # Blocked tiles of each pattern's plan (tiles of 64 rows).
            rec["plan"] = {}
            for tag, (pp, ii) in (("orig", (ptr, ind)), ("reordered", (p2, i2))):
                plan = sporder.spmm_plan(pp, ii, ctx=ctx)
                rec["plan"][tag] = dict(plan.info)
                plan.close()
        rec["spmm"] = {}
        for N in (widths or WIDTHS[name]):
            gen = torch.Generator(device=dev).manual_seed(42)
            B = torch.randn((n, N), generator=gen, dtype=torch.float32, device=dev)
            by = spmm_bytes(n, nnz, N)
            for algo in algos:
                to = _spmm_ms(sporder, ctx, ptr, ind, val, B, algo, spmm_iters, spmm_warmup)
                tr = _spmm_ms(sporder, ctx, p2, i2, v2, B, algo, spmm_iters, spmm_warmup)
                rec["spmm"][f"{N}/{algo}"] = {
                    "orig_ms": round(to, 4), "reordered_ms": round(tr, 4),
                    "orig_gbs": round(by / to / 1e6, 1), "reordered_gbs": round(by / tr / 1e6, 1)}
                print(f"[{name}] N={N} {algo}: original {to:.4f} ms, reordered {tr:.4f} ms "
                      f"({by / tr / 1e6:.0f} GB/s)", file=sys.stderr, flush=True)
            del B
    return rec


# Chunk tiers of the csg sketch (csrc/csg_local.hip chunk_tier: kT1Keys,
# kT1Rows, kT2SharedKeys for symmetric input, kT2Rows): a chunk of E nonzeros
# and R rows runs in tier 1 if E <= 16384 and R <= 1024, in tier 2 if
# E <= 28672 and R <= 4096, else on the global path.
TIER1_KEYS, TIER1_ROWS, TIER2_KEYS, TIER2_ROWS = 16384, 1024, 28672, 4096


def candidate_stats(ptr, ind, chunk: int, M: int) -> dict:
    """Stream length and distinct candidates of every row's chunk-restricted
    stream (reference sporder/src/common/chunk_similarity_top_k.cu:53-83:
    for each column of row r, the other rows of r's chunk in that column).

    Distinct candidates of row r = nonzeros of row r of A_q A_q^T without the
    diagonal, A_q the rows of r's chunk; stream length = the sum over r's
    columns of (rows of the chunk in that column) - 1.  ``items_by_tier``
    splits the stream lengths by the tier that runs the row's chunk for a
    symmetric input (the table above)."""
    import scipy.sparse as sp

    ptr = np.asarray(ptr, np.int64)
    ind = np.asarray(ind, np.int64)
    n, nnz = ptr.shape[0] - 1, ind.shape[0]
    A = sp.csr_matrix((np.ones(nnz, np.int32), ind, ptr), shape=(n, n))
    rows = np.repeat(np.arange(n), np.diff(ptr))
    key = ind * ((n + chunk - 1) // chunk) + rows // chunk
    _, inv, cnt = np.unique(key, return_inverse=True, return_counts=True)
    length = np.bincount(rows, weights=cnt[inv] - 1, minlength=n).astype(np.int64)
    distinct = np.zeros(n, np.int64)
    for q0 in range(0, n, chunk):
        sub = A[q0:min(q0 + chunk, n)]
        prod = (sub @ sub.T).tocsr()
        prod.setdiag(0)
        prod.eliminate_zeros()
        distinct[q0:q0 + sub.shape[0]] = np.diff(prod.indptr)
    busy = length > 0
    fits = busy & (distinct <= M)
    top = np.argsort(length, kind="stable")[::-1][:5]
    starts = np.arange(0, n, chunk)
    E = ptr[np.minimum(starts + chunk, n)] - ptr[starts]
    R = np.minimum(starts + chunk, n) - starts
    tier = np.where((E <= TIER1_KEYS) & (R <= TIER1_ROWS), 1,
                    np.where((E <= TIER2_KEYS) & (R <= TIER2_ROWS), 2, 3))
    by_tier = np.bincount(tier[np.arange(n) // chunk], weights=length, minlength=4)
    return {
        "M": M, "rows_with_items": int(busy.sum()), "rows_within_M": int(fits.sum()),
        "items": int(length.sum()), "items_within_M": int(length[fits].sum()),
        "rows_at_M": int((distinct == M).sum()), "rows_at_M_plus_1": int((distinct == M + 1).sum()),
        "items_by_tier": {"tier1": int(by_tier[1]), "tier2": int(by_tier[2]),
                          "global": int(by_tier[3])},
        "longest": [{"row": int(r), "items": int(length[r]), "distinct": int(distinct[r])}
                    for r in top],
    }


def run_stats(ptr, ind, block_bits: int = 10) -> dict:
    """The rows the permutation apply lists for its long-row stage (more than
    2G entries, G = the mean row length rounded up to a power of two in
    [4, 64]) and their runs of equal column block c >> block_bits: under an
    order that keeps every column inside its block (csg and cg with chunks of
    2^block_bits) the apply sorts runs, not rows.  Host only."""
    ptr = np.asarray(ptr, np.int64)
    ind = np.asarray(ind, np.int64)
    n, nnz = ptr.shape[0] - 1, ind.shape[0]
    G = 4
    while G < 64 and G * n < nnz:
        G <<= 1
    lens = np.diff(ptr)
    long_rows = lens > 2 * G
    rows = np.repeat(np.arange(n), lens)
    sel = long_rows[rows]
    key = rows[sel] * ((n >> block_bits) + 1) + (ind[sel] >> block_bits)
    cut = np.flatnonzero(np.diff(key) != 0) + 1
    runs = np.diff(np.concatenate([[0], cut, [key.shape[0]]])) if key.size else np.zeros(0)
    out = {"G": G, "long_rows": int(long_rows.sum()), "long_entries": int(lens[long_rows].sum()),
           "runs": int(runs.shape[0]), "mean_run": float(runs.mean()) if runs.size else 0.0,
           "max_run": int(runs.max()) if runs.size else 0}
    for t in (1, 2, 8, 64):
        out[f"runs_le_{t}"] = float((runs <= t).mean()) if runs.size else 1.0
        out[f"entries_in_runs_le_{t}"] = (float(runs[runs <= t].sum() / runs.sum())
                                          if runs.size else 1.0)
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--cfg", default="C1,C2,C3,C4,C5")
    ap.add_argument("--no-spmm", action="store_true")
    ap.add_argument("--algos", default="row_split,merge_path,plan")
    ap.add_argument("--repeats", type=int, default=3)
    ap.add_argument("--cg", action="store_true", help="also time sporder-cg once")
    ap.add_argument("--candidates", action="store_true",
                    help="host only: rows whose candidate streams fit the sketch")
    ap.add_argument("--widths", default=None, help="SpMM widths, e.g. 32,256 (default: "
                    "the configuration's own)")
    ap.add_argument("--spmm-iters", type=int, default=20)
    ap.add_argument("--spmm-warmup", type=int, default=5)
    ap.add_argument("--calibrate", type=int, default=0, metavar="BYTES",
                    help="one library copy-kernel launch over BYTES before each "
                    "configuration (the reference dispatch of a --pmc run)")
    ap.add_argument("--cache", default=None, metavar="DIR",
                    help="keep generated inputs as DIR/<config>.npz and reuse them")
    ap.add_argument("--runs", action="store_true",
                    help="host only: long rows of the permutation apply and their block runs")
    args = ap.parse_args(argv)

    if args.runs:
        gens = generators()
        for name in args.cfg.split(","):
            ptr, ind = gens[name]()[:2]
            print(json.dumps({"config": name, **run_stats(ptr, ind)}), flush=True)
        return 0

    if args.candidates:
        gens = generators()
        for name in args.cfg.split(","):
            ptr, ind = gens[name]()[:2]
            n, nnz = ptr.shape[0] - 1, ind.shape[0]
            k = min(256, max(16, nnz // n))  # csg defaults: k, oversampling 4, chunk 1024
            M = ((4 * k + 31) // 32) * 32
            rec = {"config": name, "n": n, "nnz": nnz, "k": k,
                   **candidate_stats(ptr, ind, 1024, M)}
            print(json.dumps(rec), flush=True)
        return 0

    import torch

    if not torch.cuda.is_available():
        print("sweep needs a ROCm GPU", file=sys.stderr)
        return 1
    for name in args.cfg.split(","):
        widths = [int(w) for w in args.widths.split(",")] if args.widths else None
        rec = measure(name, spmm=not args.no_spmm, algos=tuple(args.algos.split(",")),
                      repeats=args.repeats, cg=args.cg, widths=widths,
                      spmm_iters=args.spmm_iters, spmm_warmup=args.spmm_warmup,
                      calibrate=args.calibrate, cache=args.cache)
        print(json.dumps(rec), flush=True)
        torch.cuda.empty_cache()
    return 0


if __name__ == "__main__":
    sys.exit(main())
