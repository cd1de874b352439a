"""Benchmark of the Chunked Greedy hot path on one MI355X.

Metric: reorder time (ms) + reordered vs original SpMM GB/s,
N=32..256, 1 GPU.  Workload: configuration C2 (planted blocks, n = 2^20,
16 nnz/row, 16,777,216 nnz), synthetic and seeded, generated on the host and
resident in HBM before timing starts.

One step = csg reorder (sporder.chunk_similarity_greedy) + symmetric
permutation apply with values (sporder.reorder) + CSR SpMM at N=128 on the
reordered matrix, without a plan (a new reordering has none; a plan is the
harness's untimed prepare step and is used for the per-launch SpMM figures
below).  W untimed steps, then K timed steps between
torch.cuda.synchronize() calls -> ms_per_step.

Reported beside it (same run):
  - reorder wall_ms, median of 5 timed calls after a 1 GiB cache flush each
    (the reference harness protocol, bench/reorder/reorder_bench/methods/
    sporder_csg.py:41-57), with the stage spans;
  - SpMM kernel time per launch (warmup 30, 100 iterations, HIP events on the
    library stream; bench/spmm/spmm_bench/batch_bench.py:229-231) for the
    original and the reordered matrix at N = 32 and 128, as algorithmic GB/s
    with B_spmm(N) = 4(n+1) + 8 nnz + 8 n N bytes;
  - value = reordered SpMM GB/s at N = 128;
  - hbm_ceiling: this library's own read, write and copy kernels over 1 GiB
    (sporder_hbm_stream, ordinary and non-temporal), the rate streaming code
    reaches on the device;
  - roofline of the dominant kernel (largest share of the step) against
    8 TB/s, and cpu_baseline: the oracle (C++/OpenMP restatement of csg and a
    CSR SpMM in the same fmaf order) on the host cores.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def spmm_bytes(n, nnz, N):
    return 4 * (n + 1) + 8 * nnz + 8 * n * N


def pmc_traffic(kernel, n, nnz):
    """HBM bytes per launch of `kernel` on this workload, from the committed
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE summary (profiles/pmc_traffic.json,
    counters scaled by a copy kernel of known size); None when absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "pmc_traffic.json")
    try:
        with open(path) as f:
            table = json.load(f)
    except (OSError, ValueError):
        return None
    rec = table.get(kernel)
    if not rec or rec.get("n") != n or rec.get("nnz") != nnz:
        return None
    return rec.get("bytes_per_launch")


def host_cpu():
    """(CPU model, os.cpu_count(), CPUs this process may run on)."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count() or 1
    return model, os.cpu_count() or 1, usable


def reorder_bytes(n, nnz, k, symmetric):
    b = 2 * (4 * (n + 1) + 4 * nnz) + 8 * n * k   # sketch: CSR + CSC reads, table write
    b += 8 * n * k + 4 * n                         # greedy: table read, order write
    if not symmetric:
        b += 2 * (4 * (n + 1) + 4 * nnz)           # transpose
    return b


def band_demo(sporder, torch, dev, ctx, iters):
    """The blocked SpMM where rows share columns: a band |i - j| <= 8 of
    n = 2^20 rows (17 nonzeros per row, values U(-1, 1) seed 1), N = 128,
    B = randn seed 42.  Per-launch times of the row-split and of the planned
    SpMM (every tile in 8-row blocks), algorithmic GB/s and the fraction of
    8 TB/s; '_check' compares the planned C with the oracle (CPU leg)."""
    from chunkedgreedy_amd import synth

    n = 1 << 20
    ptr_h, ind_h, _ = synth.band(n, 8)
    val_h = np.random.default_rng(1).uniform(-1, 1, ind_h.shape[0]).astype(np.float32)
    nnz = int(ind_h.shape[0])
    p, i, v = (torch.from_numpy(a).to(dev) for a in (ptr_h, ind_h, val_h))
    gen = torch.Generator(device=dev).manual_seed(42)
    B = torch.randn((n, 128), generator=gen, dtype=torch.float32, device=dev)
    t0 = time.perf_counter()
    plan = sporder.spmm_plan(p, i, ctx=ctx)
    plan_ms = (time.perf_counter() - t0) * 1e3
    out = torch.empty((n, 128), dtype=torch.float32, device=dev)

    def timed(pl):
        for _ in range(30):
            sporder.spmm_csr(p, i, v, B, out=out, ctx=ctx, plan=pl)
        tot = 0.0
        for _ in range(iters):
            tot += sporder.spmm_csr(p, i, v, B, out=out, ctx=ctx, plan=pl)[1]
        return tot / iters

    t_rs = timed(None)
    ref = out.clone()
    t_bl = timed(plan)
    same = bool(torch.equal(out.view(torch.int32), ref.view(torch.int32)))
    bts = spmm_bytes(n, nnz, 128)
    res = {"workload": "band |i-j|<=8, n=2^20, N=128", "n": n, "nnz": nnz,
           "plan": plan.info, "plan_ms": round(plan_ms, 2),
           "rowsplit_ms": round(t_rs, 4), "blocked_ms": round(t_bl, 4),
           "blocked_gbs": round(bts / t_bl / 1e6, 1),
           "frac": round(bts / t_bl / 1e6 / HBM_PEAK_GBS, 4),
           "rowsplit_frac": round(bts / t_rs / 1e6 / HBM_PEAK_GBS, 4),
           "bit_exact_vs_rowsplit": same,
           "traffic": pmc_traffic("spmm_block_band_n128", n, nnz)}
    log(f"band demo {res}")
    C_h = out.cpu().numpy()
    B_h = B.cpu().numpy()

    def check():
        import oracle

        want = oracle.spmm_csr(ptr_h, ind_h, val_h, B_h)
        return bool(np.array_equal(C_h.view(np.uint32), want.view(np.uint32)))

    res["_check"] = check
    return res


def copy_rate(torch, dev):
    """Device-to-device copy rate of a 1 GiB tensor (bytes read + written per
    second, median of 5): the practical HBM ceiling beside the 8 TB/s peak."""
    src = torch.ones((1 << 30) // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    ts = []
    for _ in range(6):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        dst.copy_(src)
        b.record()
        b.synchronize()
        ts.append(a.elapsed_time(b))
    del src, dst
    return round(2 * (1 << 30) / statistics.median(ts[1:]) / 1e6, 1)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--rows", type=int, default=1 << 20, help="C2 row count (default 2^20)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--spmm-iters", type=int, default=100)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="first run one launch of this library's copy kernel over BYTES (a "
                         "kernel of known traffic for scaling rocprofv3 FETCH_SIZE / "
                         "WRITE_SIZE)")
    ap.add_argument("--only-spmm", action="store_true",
                    help="profiler pass: one reorder, then --spmm-iters SpMMs at N=128 on the "
                         "reordered matrix; prints no JSON line")
    ap.add_argument("--read-calibration", type=int, default=0, metavar="BYTES",
                    help="first run one reduction over BYTES (a pure read of known traffic)")
    ap.add_argument("--only-band", action="store_true",
                    help="profiler pass: the band demo's SpMMs only (row-split and blocked); "
                         "prints no JSON line")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the Chunked Greedy path has no multi-GPU "
              "execution in this build (its chunks would shard by row range, one range "
              "per GPU)", file=sys.stderr)
        sys.exit(2)

    import torch

    from chunkedgreedy_amd import sporder, synth

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.copy_calibration > 0:
        # One launch of this library's copy kernel (stream_copy_kernel<false>)
        # over the given bytes: the reference dispatch of a --pmc run.
        from chunkedgreedy_amd.sweep import calibration_copy

        calibration_copy(args.copy_calibration, sporder.Context())
        log(f"copy calibration: {args.copy_calibration} bytes read + written")
    if args.read_calibration > 0:
        src = torch.ones(args.read_calibration // 4, dtype=torch.float32, device=dev)
        total = float(src.sum())
        log(f"read calibration: {args.read_calibration} bytes read (sum {total:.0f})")
        del src
    if args.only_band:
        band_demo(sporder, torch, dev, sporder.Context(), args.spmm_iters)
        torch.cuda.synchronize()
        return

    n_rows = args.rows
    blocks = n_rows // 64
    t0 = time.time()
    ptr_h, ind_h, val_h = synth.config2(seed=args.seed, n=n_rows, blocks=blocks)
    n = ptr_h.shape[0] - 1
    nnz = int(ind_h.shape[0])
    is_sym = synth.is_pattern_symmetric(ptr_h, ind_h)
    log(f"generated C2 n={n} nnz={nnz} symmetric={is_sym} in {time.time() - t0:.1f}s")

    ptr = torch.from_numpy(ptr_h).to(dev)
    ind = torch.from_numpy(ind_h).to(dev)
    val = torch.from_numpy(val_h).to(dev)
    gen = torch.Generator(device=dev).manual_seed(42)
    B128 = torch.randn((n, 128), generator=gen, dtype=torch.float32, device=dev)
    gen = torch.Generator(device=dev).manual_seed(42)
    B32 = torch.randn((n, 32), generator=gen, dtype=torch.float32, device=dev)
    ctx = sporder.Context()
    out128 = torch.empty((n, 128), dtype=torch.float32, device=dev)

    def step():
        """csg reorder, P A P^T with values, SpMM at N=128 on the reordered
        matrix (row-split, no plan: the step makes a new pattern)."""
        order = sporder.chunk_similarity_greedy(ptr, ind, is_symmetric=is_sym, ctx=ctx)
        p2, i2, v2 = sporder.reorder(ptr, ind, order, val=val, symmetric=True, ctx=ctx)
        sporder.spmm_csr(p2, i2, v2, B128, out=out128, ctx=ctx)
        return order, (p2, i2, v2)

    # The reordered pattern (the same each step: csg is deterministic) and its
    # SpMM plan for the per-launch figures, built once outside the timed
    # region (the harness's prepare step).
    order, (p2, i2, v2) = step()
    t_plan = time.perf_counter()
    plan = sporder.spmm_plan(p2, i2, ctx=ctx)
    plan_ms = (time.perf_counter() - t_plan) * 1e3
    log(f"spmm plan of the reordered C2: {plan.info} in {plan_ms:.1f} ms")

    if args.only_spmm:
        for _ in range(args.spmm_iters):
            sporder.spmm_csr(p2, i2, v2, B128, out=out128, ctx=ctx, plan=plan)
        torch.cuda.synchronize()
        log(f"only-spmm: {args.spmm_iters} SpMMs at N=128 on the reordered matrix")
        return

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        order, reordered = step()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / max(args.steps, 1)
    log(f"step {ms_per_step:.3f} ms")

    # Reorder protocol: flush, timed call with timing; median of 5.
    flush = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    walls, spans = [], []
    for _ in range(5):
        flush.zero_()
        torch.cuda.synchronize()
        _, timing = sporder.chunk_similarity_greedy(ptr, ind, is_symmetric=is_sym,
                                                    with_timing=True, ctx=ctx)
        walls.append(timing["wall_ms"])
        spans.append(timing)
    del flush
    med = statistics.median(walls)
    span = spans[walls.index(med)] if med in walls else spans[0]
    _, stats = sporder.chunk_similarity_greedy(ptr, ind, is_symmetric=is_sym, with_stats=True,
                                               ctx=ctx)
    log(f"reorder wall median {med:.3f} ms spans {span}")

    # Permutation apply timing (events around the call).
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    perm_ms = []
    for _ in range(5):
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        sporder.reorder(ptr, ind, order, val=val, symmetric=True, ctx=ctx)
        perm_ms.append((time.perf_counter() - t1) * 1e3)
    perm_med = statistics.median(perm_ms)

    # SpMM per-launch kernel time, original vs reordered, each through its
    # plan (the harness's prepare step, untimed).
    p2, i2, v2 = reordered
    plan_orig = sporder.spmm_plan(ptr, ind, ctx=ctx)

    def spmm_ms(p, i, v, B, pl=None):
        out = torch.empty((n, B.shape[1]), dtype=torch.float32, device=dev)
        for _ in range(30):
            sporder.spmm_csr(p, i, v, B, out=out, ctx=ctx, plan=pl)
        tot = 0.0
        for _ in range(args.spmm_iters):
            _, ms = sporder.spmm_csr(p, i, v, B, out=out, ctx=ctx, plan=pl)
            tot += ms
        return tot / args.spmm_iters

    spmm = {}
    for N, B in ((32, B32), (128, B128)):
        t_orig = spmm_ms(ptr, ind, val, B, plan_orig)
        t_re = spmm_ms(p2, i2, v2, B, plan)
        bts = spmm_bytes(n, nnz, N)
        spmm[str(N)] = {
            "orig_ms": round(t_orig, 4), "reordered_ms": round(t_re, 4),
            "orig_gbs": round(bts / t_orig / 1e6, 1),
            "reordered_gbs": round(bts / t_re / 1e6, 1),
            "bytes": bts,
        }
        log(f"spmm N={N}: orig {t_orig:.3f} ms, reordered {t_re:.3f} ms")

    # Gather ceiling of the same kernel at the same shape (n rows, 16 nonzeros
    # per row, N = 128): columns drawn uniformly from the first 8192 rows (the
    # 4 MiB of B that one XCD's L2 holds), from the first 65536 and 262144 rows
    # (32 and 128 MiB of B: past the L2s, inside the 256 MB Infinity Cache) and
    # from all n rows (C2's pattern: 512 MiB of B, every gather misses L2).
    ceiling = {}
    gen = torch.Generator(device=dev).manual_seed(7)
    cptr = torch.arange(0, nnz + 1, 16, dtype=torch.int32, device=dev)
    cval = torch.rand(nnz, generator=gen, device=dev)
    spans = (("l2_resident_cols", 8192), ("b_32mib_cols", 65536), ("b_128mib_cols", 262144),
             ("uniform_cols", n))
    for label, col_span in spans:
        col_span = min(col_span, n)
        cind = torch.randint(0, col_span, (nnz,), generator=gen, device=dev, dtype=torch.int32)
        cind = cind.view(n, 16).sort(dim=1).values.reshape(-1).contiguous()
        t_c = spmm_ms(cptr, cind, cval, B128)
        ceiling[label] = {"ms": round(t_c, 4),
                          "gbs": round(spmm_bytes(n, nnz, 128) / t_c / 1e6, 1),
                          "gather_gbs": round(4.0 * nnz * 128 / t_c / 1e6, 1)}
        del cind
    log(f"spmm ceiling {ceiling}")
    band = band_demo(sporder, torch, dev, ctx, args.spmm_iters)
    copy_gbs = copy_rate(torch, dev)
    from chunkedgreedy_amd.hbm import hbm_ceiling

    ceiling_hbm = hbm_ceiling(1 << 30, 10, ctx=ctx)
    log(f"hbm ceiling (own kernels, 1 GiB) {ceiling_hbm}")
    best_read = max(ceiling_hbm["read"]["gbs"], ceiling_hbm["read"]["gbs_nt"])
    band["frac_of_read_ceiling"] = round(band["blocked_gbs"] / best_read, 4)

    k_used = stats["k_used"]
    # Dominant kernel of the step: compare the stage spans with the SpMM.
    stage = {
        "csg_sketch": span["similarity_ms"],
        "csg_greedy": span["chunk_greedy_ms"],
        "csr2csc": span["csr2csc_ms"],
        "spmm_rowsplit_n128": spmm["128"]["reordered_ms"],
    }
    dom = max(stage, key=stage.get)
    algo_bytes = {
        "csg_sketch": 2 * (4 * (n + 1) + 4 * nnz) + 8 * n * k_used,
        "csg_greedy": 8 * n * k_used + 4 * n,
        "csr2csc": 2 * (4 * (n + 1) + 4 * nnz),
        "spmm_rowsplit_n128": spmm_bytes(n, nnz, 128),
    }
    achieved = algo_bytes[dom] / (stage[dom] * 1e-3) / 1e9
    roofline = {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": pmc_traffic(dom, n, nnz),
                "algorithmic_bytes": algo_bytes[dom], "avg_ms": round(stage[dom], 4)}
    spmm_ach = spmm["128"]["reordered_gbs"]
    roofline_spmm = {"kernel": "spmm_rowsplit_n128", "bound": "hbm", "achieved": spmm_ach,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(spmm_ach / HBM_PEAK_GBS, 4)}
    reorder_gbs = reorder_bytes(n, nnz, k_used, is_sym) / (med * 1e-3) / 1e9

    cpu = None
    if not args.no_cpu:
        import oracle

        # Every usable host CPU, unless OMP_NUM_THREADS sets the allotment (the
        # GPU boxes set it to their per-GPU CPU share).
        model, ncpu, usable = host_cpu()
        threads = usable
        if os.environ.get("OMP_NUM_THREADS", "").isdigit():
            threads = max(1, min(usable, int(os.environ["OMP_NUM_THREADS"])))
        oracle.set_num_threads(threads)
        log(f"cpu baseline on {threads} threads ({model}; {usable} usable of {ncpu})")
        cpu_reorder = []
        for _ in range(5):
            t1 = time.perf_counter()
            o_order, _ = oracle.chunk_similarity_greedy(ptr_h, ind_h, is_symmetric=is_sym)
            cpu_reorder.append((time.perf_counter() - t1) * 1e3)
        parity = bool(np.array_equal(o_order, order.cpu().numpy()))
        B_h = B128.cpu().numpy()
        p2h, i2h, v2h = (x.cpu().numpy() for x in reordered)
        op, oi, ov = oracle.reorder(ptr_h, ind_h, o_order, val=val_h, symmetric=True)
        apply_parity = bool(np.array_equal(op, p2h) and np.array_equal(oi, i2h)
                            and np.array_equal(ov.view(np.uint32), v2h.view(np.uint32)))
        cpu_spmm = []
        for _ in range(5):
            t1 = time.perf_counter()
            c_ref = oracle.spmm_csr(p2h, i2h, v2h, B_h)
            cpu_spmm.append((time.perf_counter() - t1) * 1e3)
        cs = statistics.median(cpu_spmm)
        # The headline SpMM (reordered C2, N = 128, B seed 42, through its
        # plan) against the oracle's stated fmaf order, bit for bit; and the
        # band demo's blocked SpMM.
        c_gpu, _ = sporder.spmm_csr(p2, i2, v2, B128, ctx=ctx, plan=plan)
        spmm_parity = bool(np.array_equal(c_gpu.cpu().numpy().view(np.uint32),
                                          c_ref.view(np.uint32)))
        del c_gpu, c_ref
        band["bit_exact_vs_cpu"] = band.pop("_check")()
        log(f"cpu parity: permutation {parity}, apply {apply_parity}, spmm {spmm_parity}")
        cpu = {"value": round(spmm_bytes(n, nnz, 128) / (cs * 1e-3) / 1e9, 2), "unit": "GB/s",
               "cores": threads, "kind": "port",
               "sample": "full C2: oracle CSR SpMM N=128 on the reordered matrix (median of 5)"
                         "; csg reorder by the oracle on full C2 (median of 5)",
               "cpu_model": model, "cpu_count": ncpu, "cpus_usable": usable,
               "reorder_ms": round(statistics.median(cpu_reorder), 2),
               "spmm_ms": round(cs, 2), "permutation_bit_exact_vs_gpu": parity,
               "reorder_apply_bit_exact_vs_gpu": apply_parity,
               "spmm_bit_exact_vs_cpu": spmm_parity}

    out = {
        "metric": "reorder time (ms) + reordered vs original SpMM GB/s, N=32..256, 1 GPU",
        "value": spmm["128"]["reordered_gbs"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": "C2 planted blocks", "n": n, "nnz": nnz, "blocks": blocks,
                   "nnz_per_row": 16, "spmm_N": [32, 128], "k": k_used,
                   "m": stats["m_used"], "chunk_size": stats["chunk_size_used"],
                   "seed": args.seed, "is_symmetric": is_sym},
        "reorder_ms": round(med, 4),
        "reorder_spans_ms": {k: round(v, 4) for k, v in span.items() if k != "wall_ms"},
        "reorder_gbs": round(reorder_gbs, 1),
        "permute_ms": round(perm_med, 4),
        "spmm": spmm,
        "csg_stats": stats,
        "roofline": roofline,
        "roofline_spmm": roofline_spmm,
        "spmm_ceiling_n128": ceiling,
        "spmm_plan_c2": {"info": plan.info, "plan_ms": round(plan_ms, 2)},
        "spmm_block_band": band,
        "hbm_copy_gbs": copy_gbs,
        "hbm_ceiling": ceiling_hbm,
        "cpu_baseline": cpu,
    }
    band.pop("_check", None)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
