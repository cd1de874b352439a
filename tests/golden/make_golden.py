"""Writes tests/golden/sketch_cases.json: known-answer cases for the
space-saving sketch, the top-k merge and the chunk-restricted stream.

The expected outputs below were worked out by hand from the rules of the
reference sketch (sporder/src/common/warp_spacesaving.cuh:31-150,
cuda_util.cuh:66-87):
  * slots fill in order s = lane*CELLS + cell;
  * eviction takes the minimum weight, ties to the smaller (cell << 5 | lane),
    and the new key inherits the evicted weight;
  * output = per-lane selection sort (strict '>', not stable), then a merge
    taking the largest head weight, ties to the smaller lane.
Each case is built so that a plausible mistake (slot-order eviction, a stable
sort, dropping the inherited weight, ties to the larger lane) changes the
answer.  fp32 sums that are not exact are computed here with numpy float32,
one addition at a time, in stream order.  Nothing here calls the oracle or
the library.

Run: python tests/golden/make_golden.py
"""

import json
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def f32_seq_sum(values):
    acc = np.float32(0.0)
    first = True
    for v in values:
        acc = np.float32(v) if first else np.float32(acc + np.float32(v))
        first = False
    return acc


def bits(x):
    return int(np.float32(x).view(np.uint32))


def stream_cases():
    cases = []
    # E1: 32 equal weights fill M=32; key 100 evicts lane 0 and inherits 1.0.
    keys = list(range(32)) + [100]
    w = [1.0] * 32 + [0.5]
    cases.append(dict(name="E1_evict_tie_lane0", m=32, k=4, keys=keys, weights=w,
                      expected=[(100, 1.5), (1, 1.0), (2, 1.0), (3, 1.0)]))
    # E2: evictions move through lanes 0, 1, 2; a returning evicted key is new.
    keys = list(range(32)) + [40, 41, 40, 0]
    w = [1.0] * 32 + [0.5, 0.5, 0.25, 2.0]
    cases.append(dict(name="E2_evict_sequence", m=32, k=4, keys=keys, weights=w,
                      expected=[(0, 3.0), (40, 1.75), (41, 1.5), (3, 1.0)]))
    # E3: CELLS=2; ties evict cell 0 of lanes 0,1,2 (keys 0,2,4), not key 1.
    keys = list(range(64)) + [100, 101, 102]
    w = [1.0] * 67
    cases.append(dict(name="E3_evict_cell_major", m=64, k=5, keys=keys, weights=w,
                      expected=[(100, 2.0), (101, 2.0), (102, 2.0), (1, 1.0), (3, 1.0)]))
    # E4: CELLS=4, one lane; selection sort of [2,1,2,3] is not stable.
    cases.append(dict(name="E4_unstable_selection_sort", m=128, k=4, keys=[0, 1, 2, 3],
                      weights=[2.0, 1.0, 2.0, 3.0],
                      expected=[(3, 3.0), (2, 2.0), (0, 2.0), (1, 1.0)]))
    # E5: fp32 sums in stream order.
    s7 = f32_seq_sum([0.1, 0.2, 0.3])
    s8 = f32_seq_sum([0.3, 0.2, 0.1])
    exp = sorted([(7, s7), (8, s8)], key=lambda t: (-float(t[1]), t[0]))
    # Equal sums would tie to the smaller lane = key 7 (lane 0 cell 0).
    cases.append(dict(name="E5_fp32_order", m=32, k=2, keys=[7, 8, 7, 8, 7, 8],
                      weights=[0.1, 0.3, 0.2, 0.2, 0.3, 0.1],
                      expected=[(int(a), float(b)) for a, b in exp],
                      expected_bits=[bits(b) for _, b in exp]))
    # E6: fewer items than k; exhausted lanes stop the merge.
    cases.append(dict(name="E6_short_output", m=64, k=8, keys=[5, 6, 7],
                      weights=[0.5, 0.25, 0.75],
                      expected=[(7, 0.75), (5, 0.5), (6, 0.25)]))
    # E7: CELLS=2, equal minima at (lane0,cell1) and (lane1,cell0): the key
    # (cell<<5|lane) picks lane 1 cell 0 (key 2) first, then key 1.
    keys = list(range(64)) + [100, 101]
    w = [1.0] * 64 + [4.0, 4.0]
    w[1] = 0.5
    w[2] = 0.5
    cases.append(dict(name="E7_evict_key_order", m=64, k=4, keys=keys, weights=w,
                      expected=[(101, 4.5), (100, 4.5), (0, 1.0), (3, 1.0)]))
    # E8: merge ties go to the smaller lane, not the larger key or weight order.
    cases.append(dict(name="E8_merge_ties", m=32, k=3, keys=[9, 4, 6], weights=[1.0, 1.0, 1.0],
                      expected=[(9, 1.0), (4, 1.0), (6, 1.0)]))
    for c in cases:
        c.setdefault("expected_bits", [bits(wt) for _, wt in c["expected"]])
        c["weights_bits"] = [bits(x) for x in c["weights"]]
    return cases


def csr_cases():
    cases = []
    # S1: star column.  Rows 1..33 hold only column 0, row 0 holds column 0,
    # rows 34..39 hold their own column.  Row 0's stream (one chunk) is rows
    # 1..33 in order, each with alpha = 2/(1+1) = 1.0; M = 32 fills with rows
    # 1..32, row 33 evicts lane 0 (row 1) and inherits 1.0.
    n = 40
    rows = [[0]] + [[0] for _ in range(1, 34)] + [[r] for r in range(34, 40)]
    ptr = [0]
    ind = []
    for r in rows:
        ind += r
        ptr.append(len(ind))
    row0_global = [(33, 2.0), (2, 1.0), (3, 1.0), (4, 1.0)]
    # Row 1's stream: rows 0, 2..33; keys 0, 2..32 fill, 33 evicts row 0.
    row1_global = [(33, 2.0), (2, 1.0), (3, 1.0), (4, 1.0)]
    # Chunk 20: row 0 sees rows 1..19 only (no eviction).
    row0_chunk20 = [(1, 1.0), (2, 1.0), (3, 1.0), (4, 1.0)]
    # Row 25 (chunk [20, 40)): rows 20..24, 26..33 share column 0.
    row25_chunk20 = [(20, 1.0), (21, 1.0), (22, 1.0), (23, 1.0)]
    cases.append(dict(name="S1_star", n=n, ptr=ptr, ind=ind, k=4, oversampling=8.0,
                      checks=[dict(chunk=n, row=0, expected=row0_global),
                              dict(chunk=n, row=1, expected=row1_global),
                              dict(chunk=20, row=0, expected=row0_chunk20),
                              dict(chunk=20, row=25, expected=row25_chunk20),
                              dict(chunk=20, row=35, expected=[])]))
    # S2: weights from row sizes and repeated columns.  Row 0 = {0,1,2};
    # row 1 = {0,1} (alpha 2/5 twice); row 2 = {2,3,4,5} (alpha 2/7 once);
    # row 3 = {0} (alpha 2/4 once).  Stream of row 0 (global): col 0 -> rows
    # 1,3; col 1 -> row 1; col 2 -> row 2.  Row 1 weight = fl(0.4 + 0.4).
    ptr = [0, 3, 5, 9, 10, 11, 12]
    ind = [0, 1, 2, 0, 1, 2, 3, 4, 5, 0, 4, 5]
    two_fifths = np.float32(2.0) / np.float32(5.0)
    w1 = np.float32(two_fifths + two_fifths)
    w2 = np.float32(2.0) / np.float32(7.0)
    exp = [(1, float(w1)), (3, 0.5), (2, float(w2))]
    cases.append(dict(name="S2_dice_weights", n=6, ptr=ptr, ind=ind, k=4, oversampling=8.0,
                      checks=[dict(chunk=6, row=0, expected=exp,
                                   expected_bits=[bits(w1), bits(0.5), bits(w2)])]))
    for c in cases:
        for chk in c["checks"]:
            chk.setdefault("expected_bits", [bits(wt) for _, wt in chk["expected"]])
    return cases


def band_kat():
    # Reference smoke matrix (sporder/tests/smoke.c:58-70): n=1000, |i-j|<=2.
    # Row 0 = {0,1,2} (|r0| = 3).  Candidates: row 1 (|.|=4) shares 3 columns,
    # alpha 2/7 added three times; row 2 (|.|=5) shares 3, alpha 2/8; row 3
    # shares 2; row 4 shares 1.  k=8, oversampling=4 -> M=32.
    a = np.float32(2.0) / np.float32(7.0)
    w1 = np.float32(np.float32(a + a) + a)
    return dict(n=1000, half_width=2, k=8, oversampling=4.0, row=0,
                expected_idx=[1, 2, 3, 4, -1, -1, -1, -1],
                expected_bits=[bits(w1), bits(0.75), bits(0.5), bits(0.25), 0, 0, 0, 0],
                fl_6_7_bits=bits(np.float32(6.0) / np.float32(7.0)))


def main():
    out = {"stream_cases": stream_cases(), "csr_cases": csr_cases(), "band_kat": band_kat()}
    (HERE / "sketch_cases.json").write_text(json.dumps(out, indent=1) + "\n")
    print("wrote", HERE / "sketch_cases.json")


if __name__ == "__main__":
    main()
