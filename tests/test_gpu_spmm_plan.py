"""GPU parity of the planned SpMM (sporder_spmm_plan_create +
sporder_spmm_csr_plan): bit-exact against the row-split (the stated fmaf
order) and the oracle, on patterns whose 64-row tiles are computed in 8-row
blocks (bands, diagonal blocks), run as row-split tiles (random, stencil,
C1), mixed with long rows, with a partial last tile and with empty rows; at
widths that take 1, 2 or 4 columns per lane (multiples of 64, 128, 256) and
widths that take the row-split (16, 32, 96).  The plan's tile decisions are
checked against a NumPy restatement of its rule."""

import numpy as np
import pytest
import torch

import oracle
from chunkedgreedy_amd import synth

pytestmark = pytest.mark.gpu


def with_values(csr, seed):
    ptr, ind = csr[0], csr[1]
    val = np.random.default_rng(seed).uniform(-1, 1, ind.shape[0]).astype(np.float32)
    return ptr, ind, val


def block_rows(n, block, in_deg, out_deg, seed):
    """Rows in blocks of `block`: in_deg columns inside the block's column
    range and out_deg uniform ones (the planted pattern in block order)."""
    rng = np.random.default_rng(seed)
    rows = np.repeat(np.arange(n), in_deg + out_deg)
    base = (rows // block) * block
    cols = np.where(np.tile(np.arange(in_deg + out_deg) < in_deg, n),
                    np.minimum(base + rng.integers(0, block, rows.size), n - 1),
                    rng.integers(0, n, rows.size))
    keys = np.unique(rows.astype(np.int64) * n + cols)
    r, c = keys // n, keys % n
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(np.bincount(r, minlength=n), out=ptr[1:])
    return ptr.astype(np.int32), c.astype(np.int32)


def random_rows(n, deg, seed, hubs=None):
    rng = np.random.default_rng(seed)
    rows = [np.repeat(np.arange(n), deg)]
    cols = [rng.integers(0, n, n * deg)]
    for r, d in (hubs or {}).items():
        rows.append(np.full(d, r))
        cols.append(rng.choice(n, d, replace=False))
    rows, cols = np.concatenate(rows), np.concatenate(cols)
    keys = np.unique(rows.astype(np.int64) * n + cols)
    r, c = keys // n, keys % n
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(np.bincount(r, minlength=n), out=ptr[1:])
    return ptr.astype(np.int32), c.astype(np.int32)


def with_repeats(csr, rows):
    """Repeat the first column of each listed row (sorted, not distinct: a
    CSR with duplicate entries, which the SpMM adds one after the other)."""
    ptr, ind = csr[0], csr[1]
    lens = np.diff(ptr)
    parts = []
    for r in range(ptr.shape[0] - 1):
        seg = ind[ptr[r]:ptr[r + 1]]
        if r in rows and seg.size:
            seg = np.concatenate([seg[:1], seg])
            lens[r] += 1
        parts.append(seg)
    p = np.zeros_like(ptr)
    np.cumsum(lens, out=p[1:])
    return p, np.concatenate(parts).astype(np.int32)


def with_empty_rows(csr, every):
    """Drop the nonzeros of every `every`-th row."""
    ptr, ind = csr[0], csr[1]
    keep = np.ones(ind.shape[0], bool)
    lens = np.diff(ptr)
    for r in range(0, ptr.shape[0] - 1, every):
        keep[ptr[r]:ptr[r + 1]] = False
        lens[r] = 0
    p = np.zeros_like(ptr)
    np.cumsum(lens, out=p[1:])
    return p, ind[keep]


MATS = {
    "band8_n8192": with_values(synth.band(8192, 8), 1),
    "band40_n4000": with_values(synth.band(4000, 40), 2),         # partial last tile
    "blocks64_n8192": with_values(block_rows(8192, 64, 28, 2, 3), 3),  # diagonal blocks
    "stencil_ordered": with_values(synth.stencil7(16, 4, scramble=False), 4),  # direct
    "random_n6000": with_values(random_rows(6000, 12, 5), 5),    # direct
    "band_hubs": with_values(synth.band(6000, 4), 6),           # replaced below
    "band_empty_rows": with_values(with_empty_rows(synth.band(3000, 6), 7), 7),
    "C1": synth.config1(11),
    # Rows 5, 70 and 1000 repeat a column: their tiles (0, 1, 15) stay on the
    # row-split, the other band tiles are blocked.
    "band_repeats": with_values(with_repeats(synth.band(2000, 8), {5, 70, 1000}), 9),
}
# A band with long rows spliced in: their tiles go to the row-split segments.
_p, _i = random_rows(6000, 0, 8, hubs={100: 900, 3000: 2000, 5999: 600})
_bp, _bi = synth.band(6000, 4)[:2]
_keys = np.unique(np.concatenate([
    np.repeat(np.arange(6000), np.diff(_bp)).astype(np.int64) * 6000 + _bi,
    np.repeat(np.arange(6000), np.diff(_p)).astype(np.int64) * 6000 + _i]))
_ptr = np.zeros(6001, np.int64)
np.cumsum(np.bincount(_keys // 6000, minlength=6000), out=_ptr[1:])
MATS["band_hubs"] = with_values((_ptr.astype(np.int32), (_keys % 6000).astype(np.int32)), 6)


def dev(*arrays):
    return [torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0") for a in arrays]


@pytest.fixture(scope="module")
def plans(sporder):
    out = {}
    for name, (ptr, ind, val) in MATS.items():
        dptr, dind, dval = dev(ptr, ind, val)
        out[name] = (dptr, dind, dval, sporder.spmm_plan(dptr, dind))
    return out


@pytest.mark.parametrize("name", sorted(MATS))
@pytest.mark.parametrize("N", [16, 32, 64, 96, 128, 192, 256])
def test_planned_spmm_equals_row_split(sporder, plans, name, N):
    dptr, dind, dval, plan = plans[name]
    n = dptr.numel() - 1
    print(f"[plan] {name} N={N} info={plan.info}", flush=True)
    gen = torch.Generator(device="cuda:0").manual_seed(N)
    B = torch.randn((n, N), generator=gen, dtype=torch.float32, device="cuda:0")
    ref, _ = sporder.spmm_csr(dptr, dind, dval, B, algo="row_split")
    C, ms = sporder.spmm_csr(dptr, dind, dval, B, plan=plan)
    assert ms >= 0.0
    assert torch.equal(C.view(torch.int32), ref.view(torch.int32))
    if N in (64, 128):
        ptr, ind, val = MATS[name]
        want = oracle.spmm_csr(ptr, ind, val, B.cpu().numpy())
        assert np.array_equal(C.cpu().numpy().view(np.uint32), want.view(np.uint32))


def plan_model(ptr, ind):
    """The plan rule restated: 8-row blocks' entries are their distinct
    columns; a 64-row tile is blocked when no row has more than 512
    nonzeros, no row holds a column twice and 2 * entries <= nonzeros."""
    n = ptr.shape[0] - 1
    out = {"tiles": (n + 63) // 64, "blocked_tiles": 0, "blocked_rows": 0, "blocked_nnz": 0,
           "entries": 0}
    for t in range(out["tiles"]):
        r0, r1 = 64 * t, min(64 * t + 64, n)
        m = int(ptr[r1] - ptr[r0])
        if m == 0 or (np.diff(ptr[r0:r1 + 1]) > 512).any():
            continue
        if any(np.unique(ind[ptr[r]:ptr[r + 1]]).size < ptr[r + 1] - ptr[r]
               for r in range(r0, r1)):
            continue
        e = sum(np.unique(ind[ptr[b]:ptr[min(b + 8, r1)]]).size for b in range(r0, r1, 8))
        if 2 * e <= m:
            out["blocked_tiles"] += 1
            out["blocked_rows"] += r1 - r0
            out["blocked_nnz"] += m
            out["entries"] += e
    return out


@pytest.mark.parametrize("name", sorted(MATS))
def test_plan_info_matches_rule(plans, name):
    ptr, ind, _ = MATS[name]
    assert plans[name][3].info == plan_model(ptr, ind)


def test_plan_blocks_where_rows_share_columns(plans):
    """Every band tile is blocked (a half-width-8 band has 24 entries per
    8-row block against 136 nonzeros), no random, stencil or C1 tile is, and
    the band tiles holding a long row are not."""
    info = {k: v[3].info for k, v in plans.items()}
    b = info["band8_n8192"]
    assert b["blocked_tiles"] == b["tiles"] == 128 and b["blocked_rows"] == 8192
    assert b["entries"] == 8192 * 3 - 16 + 8 * 0  # 24 per interior block, 16 at each end
    assert info["band40_n4000"]["blocked_tiles"] == info["band40_n4000"]["tiles"]
    for name in ("random_n6000", "stencil_ordered", "C1"):
        assert info[name]["blocked_tiles"] == 0, name
    h = info["band_hubs"]
    assert h["blocked_tiles"] == h["tiles"] - len({100 // 64, 3000 // 64, 5999 // 64})
    d = info["band_repeats"]
    assert d["blocked_tiles"] == d["tiles"] - 3


def test_plan_rejects_other_matrix(sporder, plans):
    dptr, dind, dval, plan = plans["band8_n8192"]
    optr, oind, oval, _ = plans["random_n6000"]
    B = torch.zeros((optr.numel() - 1, 64), dtype=torch.float32, device="cuda:0")
    with pytest.raises(ValueError):
        sporder.spmm_csr(optr, oind, oval, B, plan=plan)
    with pytest.raises(ValueError):
        sporder.spmm_csr(dptr, dind, dval, torch.zeros((8192, 64), device="cuda:0"), plan=plan,
                         algo="merge_path")
