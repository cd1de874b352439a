"""HBM ceiling of the device, measured with this library's own streaming
kernels (``sporder_hbm_stream``): a pure read, a pure write and a copy, with
ordinary and non-temporal accesses.  The HBM-bound kernels of the path (the
SpMM, the permutation apply) are quoted against the 8 TB/s peak; these rates
say what streaming code reaches on the same device.

    python -m chunkedgreedy_amd.hbm [--mib 1024] [--iters 10]

prints one JSON object {read, write, copy} of {"gbs", "gbs_nt", "ms", "ms_nt"}
(bytes moved per second: the buffer size for read and write, twice it for a
copy).
"""

from __future__ import annotations

import argparse
import ctypes
import json

from . import _lib


def hbm_ceiling(nbytes: int = 1 << 30, iters: int = 10, ctx=None, device="cuda:0") -> dict:
    """Mean per-launch rates of the three streaming kernels over `nbytes`
    buffers (a multiple of 16)."""
    import torch

    from .sporder import Context

    if nbytes <= 0 or nbytes % 16:
        raise ValueError("nbytes must be a positive multiple of 16")
    ctx = ctx or Context()
    lib = _lib.load()
    src = torch.ones(nbytes // 4, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    out = {}
    for name, op, moved in (("read", _lib.STREAM_READ, nbytes),
                            ("write", _lib.STREAM_WRITE, nbytes),
                            ("copy", _lib.STREAM_COPY, 2 * nbytes)):
        rec = {}
        for nt in (0, 1):
            ms = ctypes.c_float()
            lib.sporder_hbm_stream(ctx.handle, op, nt, dst.data_ptr(), src.data_ptr(), nbytes,
                                   iters, ctypes.byref(ms))
            suffix = "_nt" if nt else ""
            rec["ms" + suffix] = round(ms.value, 4)
            rec["gbs" + suffix] = round(moved / (ms.value * 1e-3) / 1e9, 1)
        out[name] = rec
    del src, dst
    return out


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--mib", type=int, default=1024, help="buffer size in MiB")
    ap.add_argument("--iters", type=int, default=10)
    args = ap.parse_args()
    print(json.dumps({"bytes": args.mib << 20, **hbm_ceiling(args.mib << 20, args.iters)}),
          flush=True)


if __name__ == "__main__":
    main()
