"""Writes one row's chunk-local candidate stream for tests/c/sketch_probe:
(int32 key, float32 weight) pairs, truncated to a multiple of 64, in the order
the csg chunk tiers feed the row's sketch -- the row's columns in CSR order,
and for each column the chunk's other rows that hold it, ascending -- with
weight 2 / (deg(row) + deg(other)) in float32.

    python tests/c/hub_stream.py C3 0 /tmp/c3_row0.bin
    tests/c/sketch_probe 0 1 file /tmp/c3_row0.bin

Row 0 of C3 is its hub (2,297,664 items): one wave's cycles per item on this
stream set C3's sketch time.
"""

import sys
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))

from chunkedgreedy_amd import synth  # noqa: E402

CONFIGS = {"C3": synth.config3, "C5": synth.config5}


def row_stream(ptr: np.ndarray, ind: np.ndarray, row: int, chunk: int = 1024):
    ptr = ptr.astype(np.int64)
    ind = ind.astype(np.int64)
    cs = (row // chunk) * chunk
    ce = min(cs + chunk, len(ptr) - 1)
    rows = np.repeat(np.arange(cs, ce), np.diff(ptr[cs:ce + 1]))
    cols = ind[ptr[cs]:ptr[ce]]
    order = np.lexsort((rows, cols))
    rows_s, cols_s = rows[order], cols[order]
    deg = np.diff(ptr)
    keys, wts = [], []
    for c in ind[ptr[row]:ptr[row + 1]]:
        lo = np.searchsorted(cols_s, c)
        hi = np.searchsorted(cols_s, c, side="right")
        rr = rows_s[lo:hi]
        rr = rr[rr != row]
        keys.append(rr.astype(np.int32))
        wts.append(np.float32(2.0) / (deg[row] + deg[rr]).astype(np.float32))
    k = np.concatenate(keys)
    w = np.concatenate(wts).astype(np.float32)
    n = (len(k) // 64) * 64
    return k[:n], w[:n]


def main(argv=None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    if len(argv) != 3 or argv[0] not in CONFIGS:
        print("usage: hub_stream.py C3|C5 ROW OUT", file=sys.stderr)
        return 1
    ptr, ind = CONFIGS[argv[0]]()[:2]
    k, w = row_stream(ptr, ind, int(argv[1]))
    print(argv[0], "row", argv[1], "items", len(k), "distinct", len(np.unique(k)))
    np.stack([k, w.view(np.int32)], axis=1).astype(np.int32).tofile(argv[2])
    return 0


if __name__ == "__main__":
    sys.exit(main())
