"""Host logic of the configuration sweep (no GPU calls)."""

import numpy as np

from chunkedgreedy_amd import sweep


def test_spmm_bytes_matches_c2_figures():
    # C2: n = 2^20, nnz = 2^24; N = 128 -> 1,212,153,860 B, N = 32 -> 406,847,492 B.
    assert sweep.spmm_bytes(1 << 20, 1 << 24, 128) == 1_212_153_860
    assert sweep.spmm_bytes(1 << 20, 1 << 24, 32) == 406_847_492


def test_widths_cover_every_config():
    assert sweep.WIDTHS == {"C1": [32], "C2": [32, 128], "C3": [32, 64, 256],
                            "C4": [16, 32, 64, 128, 256], "C5": [128],
                            "C2r": [128], "C4n": [32], "RGG20": [32, 128], "C5d": [128]}
    assert set(sweep.generators()) == set(sweep.WIDTHS)


def test_main_needs_a_gpu(monkeypatch):
    import torch

    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    assert sweep.main(["--cfg", "C1"]) == 1


def test_candidate_stats_against_brute_force():
    """Stream lengths and distinct candidates of every row, against a direct
    enumeration of each row's chunk-restricted stream."""
    import numpy as np

    from chunkedgreedy_amd import synth

    ptr, ind = synth.config1(3)[:2]
    ptr, ind = ptr[:601].copy(), ind[:ptr[600]].copy()  # the first 600 rows
    ind = ind % 600
    order = np.lexsort((ind, np.repeat(np.arange(600), np.diff(ptr))))
    ind = ind[order]
    keep = np.ones(ind.size, bool)
    rows = np.repeat(np.arange(600), np.diff(ptr))
    keep[1:] = (ind[1:] != ind[:-1]) | (rows[1:] != rows[:-1])
    lens = np.bincount(rows[keep], minlength=600)
    ind = ind[keep]
    ptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    chunk, M = 64, 8
    st = sweep.candidate_stats(ptr, ind, chunk, M)
    cols = [set(ind[ptr[r]:ptr[r + 1]].tolist()) for r in range(600)]
    length, distinct = [], []
    for r in range(600):
        cs = (r // chunk) * chunk
        items = [s for c in ind[ptr[r]:ptr[r + 1]] for s in range(cs, min(cs + chunk, 600))
                 if s != r and c in cols[s]]
        length.append(len(items))
        distinct.append(len(set(items)))
    length, distinct = np.array(length), np.array(distinct)
    busy = length > 0
    assert st["rows_with_items"] == busy.sum()
    assert st["rows_within_M"] == (busy & (distinct <= M)).sum()
    assert st["items"] == length.sum()
    assert sum(st["items_by_tier"].values()) == length.sum()
    # 600 rows of at most 64 nonzeros in chunks of 64 rows: every chunk fits tier 1
    assert st["items_by_tier"]["tier1"] == length.sum()
    assert st["items_within_M"] == length[busy & (distinct <= M)].sum()
    assert st["rows_at_M"] == (distinct == M).sum()
    assert st["longest"][0]["items"] == length.max()


def test_generate_cache_round_trip(tmp_path, monkeypatch):
    """generate() writes the input once and reads it back unchanged."""
    calls = []

    def fake():
        calls.append(1)
        return (np.array([0, 1, 2], np.int32), np.array([1, 0], np.int32),
                np.array([0.5, -0.25], np.float32))

    monkeypatch.setattr(sweep, "generators", lambda: {"X": fake})
    a = sweep.generate("X", str(tmp_path))
    b = sweep.generate("X", str(tmp_path))
    assert len(calls) == 1
    for u, v in zip(a, b):
        assert u.dtype == v.dtype and np.array_equal(u, v)


def test_candidate_items_by_tier():
    """Chunks of 10, 20 and 30 nonzeros per row (1024 rows each: 10,240,
    20,480 and 30,720 nonzeros) fall in tier 1, tier 2 and the global path;
    each chunk's stream length is sum_c cnt(c) (cnt(c) - 1) over its columns'
    counts cnt(c)."""
    import numpy as np

    rng = np.random.default_rng(7)
    n, chunk = 3072, 1024
    rows = []
    for r in range(n):
        deg = 10 * (r // chunk + 1)
        rows.append(np.sort(rng.choice(n, deg, replace=False)))
    ptr = np.concatenate([[0], np.cumsum([len(x) for x in rows])]).astype(np.int32)
    ind = np.concatenate(rows).astype(np.int32)
    st = sweep.candidate_stats(ptr, ind, chunk, 128)
    want = []
    for q in range(3):
        cnt = np.bincount(ind[ptr[q * chunk]:ptr[(q + 1) * chunk]], minlength=n).astype(np.int64)
        want.append(int((cnt * (cnt - 1)).sum()))
    assert st["items_by_tier"] == {"tier1": want[0], "tier2": want[1], "global": want[2]}
    assert st["items"] == sum(want)
