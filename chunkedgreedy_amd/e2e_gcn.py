"""End-to-end 2-layer GCN on a reordered graph.

Counterpart of the reference experiment experiments/e2e_gcn.py:34-156 and its
permutation timing experiments/perm_time.py:1-16, with this library's CSR SpMM
(``sporder.spmm_csr``) as the sparse kernel:

  total_ms = reorder_ms + perm_ms + prep_ms + epochs * epoch_ms

- reorder_ms: the reorder's own wall_ms (sporder-csg or sporder-cg);
- perm_ms: the GPU symmetric permutation P A P^T of the pattern
  (``sporder.reorder(symmetric=True)``) plus the feature and label gathers
  X[perm], y[perm];
- prep_ms: the kernel's preprocessing (none for CSR: the values array of ones
  and the degree scaling, built on the GPU);
- epoch_ms: one full-batch forward + backward + Adam step.

The model (experiments/e2e_gcn.py:107-133): A is the pattern with values 1,
the normalisation D^-1/2 A D^-1/2 is applied around the SpMM as
op(x) = d^-1/2 * (A @ (d^-1/2 * x)); h1 = relu(op(X W1)), z = op(h1) W2,
cross-entropy against uniform random labels, Adam (lr 0.01).  A is symmetric,
so the backward of op is op itself: 4 SpMMs of width `hidden` per epoch.

With --fused-scaling the operator is one call of
``sporder.spmm_csr_scaled`` (the two d^-1/2 products applied inside the
SpMM: the same values bit for bit, without the two elementwise passes); the
default keeps the reference driver's three steps.

Usage:  python -m chunkedgreedy_amd.e2e_gcn [--nodes N] [--epochs E] ...
prints one JSON record per ordering (ORIGIN and sporder-csg by default;
sporder-cg on request).
"""

from __future__ import annotations

import argparse
import json
import sys
import time

import numpy as np


def _sync_ms(torch, t0: float) -> float:
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3


class GraphOp:
    """x -> d^-1/2 * (A @ (d^-1/2 * x)) on one GPU, timing each SpMM.  With
    `fused` one scaled SpMM call (bit-identical to the three steps)."""

    def __init__(self, ptr, ind, ctx=None, fused=False):
        import torch

        from chunkedgreedy_amd import sporder

        self.torch = torch
        self.sporder = sporder
        self.ptr, self.ind, self.ctx = ptr, ind, ctx
        self.val = torch.ones(ind.numel(), dtype=torch.float32, device=ind.device)
        deg = (ptr[1:] - ptr[:-1]).to(torch.float32).clamp_min(1.0)
        self.dinv = deg.rsqrt().unsqueeze(1)
        self.fused = fused
        # The fused call's column scales per nonzero, d^-1/2[ind], once.
        self.nz_scale = self.dinv.view(-1)[ind.long()] if fused else None
        self.spmm_ms = 0.0

    def __call__(self, x):
        if self.fused:
            out, ms = self.sporder.spmm_csr_scaled(self.ptr, self.ind, self.val, x.contiguous(),
                                                   row_scale=self.dinv.view(-1),
                                                   nz_col_scale=self.nz_scale, ctx=self.ctx)
            self.spmm_ms += ms
            return out
        out, ms = self.sporder.spmm_csr(self.ptr, self.ind, self.val,
                                        (self.dinv * x).contiguous(), ctx=self.ctx)
        self.spmm_ms += ms
        return self.dinv * out


def _spmm_fn():
    import torch

    class SpMMFn(torch.autograd.Function):
        """Autograd wrapper; A is symmetric, so d(op x)/dx^T g = op(g)."""

        @staticmethod
        def forward(ctx, x, op):
            ctx.op = op
            return op(x)

        @staticmethod
        def backward(ctx, g):
            return ctx.op(g.contiguous()), None

    return SpMMFn


def train(ptr, ind, X, y, *, hidden: int, classes: int, epochs: int, warmup: int = 3,
          seed: int = 0, ctx=None, fused: bool = False) -> dict:
    """Train the 2-layer GCN for `epochs` timed epochs after `warmup` untimed
    ones; returns per-epoch times, SpMM time per epoch and the losses."""
    import torch
    import torch.nn.functional as F

    t0 = time.perf_counter()
    op = GraphOp(ptr, ind, ctx=ctx, fused=fused)
    prep_ms = _sync_ms(torch, t0)
    SpMMFn = _spmm_fn()
    torch.manual_seed(seed)
    W1 = torch.nn.Linear(X.shape[1], hidden).to(X.device)
    W2 = torch.nn.Linear(hidden, classes).to(X.device)
    opt = torch.optim.Adam(list(W1.parameters()) + list(W2.parameters()), lr=0.01)

    def epoch():
        opt.zero_grad()
        h1 = F.relu(SpMMFn.apply(W1(X), op))
        z = W2(SpMMFn.apply(h1, op))
        loss = -F.log_softmax(z, 1).gather(1, y[:, None]).mean()
        loss.backward()
        opt.step()
        return loss

    losses = []
    for _ in range(warmup):
        losses.append(float(epoch().detach()))
    op.spmm_ms = 0.0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    timed = []
    for _ in range(epochs):
        timed.append(epoch())
    train_ms = _sync_ms(torch, t0)
    losses += [float(v.detach()) for v in timed]
    return {"prep_ms": prep_ms, "epoch_ms": train_ms / max(epochs, 1),
            "spmm_ms_per_epoch": op.spmm_ms / max(epochs, 1), "train_ms": train_ms,
            "losses": losses}


def permute_graph(ptr, ind, X, y, order, ctx=None):
    """P A P^T of the pattern and the gathered features and labels
    (experiments/perm_time.py:1-16: sporder.reorder + X[perm])."""
    from chunkedgreedy_amd import sporder

    p2, i2 = sporder.reorder(ptr, ind, order, symmetric=True, ctx=ctx)
    perm = order.long()
    return p2, i2, X[perm], y[perm]


def run(ptr_h, ind_h, *, features: int, hidden: int, classes: int, epochs: int,
        orders=("ORIGIN", "sporder-csg"), seed: int = 0, fused: bool = False) -> list[dict]:
    import torch

    from chunkedgreedy_amd import sporder

    dev = torch.device("cuda:0")
    n = ptr_h.shape[0] - 1
    ptr = torch.from_numpy(np.ascontiguousarray(ptr_h, np.int32)).to(dev)
    ind = torch.from_numpy(np.ascontiguousarray(ind_h, np.int32)).to(dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    X0 = torch.randn(n, features, device=dev, generator=g)
    y0 = torch.randint(0, classes, (n,), device=dev, generator=g)
    ctx = sporder.Context()
    # Untimed: the first allocations of the values and degree arrays would
    # otherwise land in the first order's prep time.
    GraphOp(ptr, ind, ctx=ctx)
    torch.cuda.synchronize()
    entries = {"sporder-csg": sporder.chunk_similarity_greedy, "sporder-cg": sporder.chunk_greedy}
    rows = []
    for name in orders:
        if name == "ORIGIN":
            reorder_ms, perm_ms = 0.0, 0.0
            ptr_u, ind_u, X, y = ptr, ind, X0, y0
        else:
            entry = entries[name]
            entry(ptr, ind, is_symmetric=True, ctx=ctx)  # warmup
            order, timing = entry(ptr, ind, is_symmetric=True, with_timing=True, ctx=ctx)
            reorder_ms = float(timing["wall_ms"])
            permute_graph(ptr, ind, X0, y0, order, ctx=ctx)  # warmup
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            ptr_u, ind_u, X, y = permute_graph(ptr, ind, X0, y0, order, ctx=ctx)
            perm_ms = _sync_ms(torch, t0)
        r = train(ptr_u, ind_u, X, y, hidden=hidden, classes=classes, epochs=epochs, seed=seed,
                  ctx=ctx, fused=fused)
        total = reorder_ms + perm_ms + r["prep_ms"] + epochs * r["epoch_ms"]
        rows.append({"order": name, "fused_scaling": fused, "n": n, "nnz": int(ind_h.shape[0]),
                     "features": features,
                     "hidden": hidden, "classes": classes, "epochs": epochs,
                     "reorder_ms": round(reorder_ms, 3), "perm_ms": round(perm_ms, 3),
                     "prep_ms": round(r["prep_ms"], 3), "epoch_ms": round(r["epoch_ms"], 3),
                     "spmm_ms_per_epoch": round(r["spmm_ms_per_epoch"], 3),
                     "train_ms": round(r["train_ms"], 2), "total_ms": round(total, 2),
                     "final_loss": r["losses"][-1]})
        del ptr_u, ind_u, X, y
    base = rows[0] if rows and rows[0]["order"] == "ORIGIN" else None
    for row in rows:
        if base is not None and row is not base:
            gain = base["epoch_ms"] - row["epoch_ms"]
            row["epoch_speedup"] = round(base["epoch_ms"] / row["epoch_ms"], 4)
            row["e2e_speedup"] = round(base["total_ms"] / row["total_ms"], 4)
            row["breakeven_epochs"] = (round((row["reorder_ms"] + row["perm_ms"]) / gain, 1)
                                       if gain > 0 else None)
    return rows


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--nodes", type=int, default=2_449_029)
    ap.add_argument("--degree", type=float, default=25.0)
    ap.add_argument("--exponent", type=float, default=2.1)
    ap.add_argument("--features", type=int, default=100)
    ap.add_argument("--hidden", type=int, default=128)
    ap.add_argument("--classes", type=int, default=47)
    ap.add_argument("--epochs", type=int, default=50)
    ap.add_argument("--seed", type=int, default=5)
    # sporder-cg's global sketch streams sum(deg(c)^2) items per row set; on a
    # Chung-Lu graph with 600K-degree hubs that is minutes, so it is opt-in.
    ap.add_argument("--orders", default="ORIGIN,sporder-csg")
    ap.add_argument("--degree-order", action="store_true",
                    help="vertices in expected-degree order (synth LOCALITY C5d) "
                    "instead of the scrambled ids of configuration C5")
    ap.add_argument("--fused-scaling", action="store_true",
                    help="apply d^-1/2 on both sides inside the SpMM (spmm_csr_scaled) "
                    "instead of as two elementwise products around it")
    args = ap.parse_args(argv)

    import torch

    if not torch.cuda.is_available():
        print("e2e_gcn needs a ROCm GPU", file=sys.stderr)
        return 1
    from chunkedgreedy_amd import synth

    t0 = time.time()
    ptr_h, ind_h, _ = synth.chung_lu(args.nodes, args.exponent, args.degree, args.seed,
                                     scramble=not args.degree_order)
    print(f"[e2e] Chung-Lu n={ptr_h.shape[0] - 1} nnz={ind_h.shape[0]} "
          f"({'degree order' if args.degree_order else 'scrambled ids'}, "
          f"{time.time() - t0:.1f}s)", file=sys.stderr, flush=True)
    for row in run(ptr_h, ind_h, features=args.features, hidden=args.hidden,
                   classes=args.classes, epochs=args.epochs,
                   orders=tuple(args.orders.split(",")), seed=args.seed,
                   fused=args.fused_scaling):
        print(json.dumps(row), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
