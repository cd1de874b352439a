"""sporder_spmm_csr_noalloc through the C ABI: equal bit for bit to
sporder_spmm_csr (row-split), on two calls in a row with the second input
smaller than the first (the static scratch keeps the first call's contents),
on a width that takes the scalar kernel, and the size rejection."""

import numpy as np
import pytest
import torch

from chunkedgreedy_amd import _lib

pytestmark = pytest.mark.gpu


def hub_csr(n, deg, hubs, seed):
    """Random rows of `deg` columns plus rows {row: nonzeros} past the
    long-row bound, so the row-split registers segments in the scratch."""
    rng = np.random.default_rng(seed)
    rows = [np.repeat(np.arange(n), deg)]
    cols = [rng.integers(0, n, size=n * deg)]
    for r, d in hubs.items():
        rows.append(np.full(d, r))
        cols.append(rng.choice(n, size=d, replace=False))
    rows, cols = np.concatenate(rows), np.concatenate(cols)
    keys = np.unique(rows.astype(np.int64) * n + cols)
    r, c = keys // n, keys % n
    ptr = np.zeros(n + 1, np.int64)
    np.cumsum(np.bincount(r, minlength=n), out=ptr[1:])
    val = rng.uniform(-1.0, 1.0, size=keys.size).astype(np.float32)
    return ptr.astype(np.int32), c.astype(np.int32), val


def to_dev(*arrays):
    return [torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0") for a in arrays]


def call_noalloc(sp, ctx, ptr, ind, val, B, out):
    n, nnz = ptr.numel() - 1, ind.numel()
    return _lib.load().sporder_spmm_csr_noalloc(
        ctx.handle, n, nnz, ptr.data_ptr(), ind.data_ptr(), val.data_ptr(), B.shape[1],
        B.data_ptr(), out.data_ptr())


@pytest.fixture(scope="module")
def ctx(sporder):
    return sporder.Context()


def check_case(sporder, ctx, ptr_h, ind_h, val_h, N, seed):
    ptr, ind, val = to_dev(ptr_h, ind_h, val_h)
    n = ptr_h.shape[0] - 1
    gen = torch.Generator(device="cuda:0").manual_seed(seed)
    B = torch.randn((n, N), generator=gen, dtype=torch.float32, device="cuda:0")
    ref, _ = sporder.spmm_csr(ptr, ind, val, B, algo="row_split", ctx=ctx)
    out = torch.full((n, N), float("nan"), dtype=torch.float32, device="cuda:0")
    rc = call_noalloc(sporder, ctx, ptr, ind, val, B, out)
    torch.cuda.synchronize()
    assert rc == 0
    assert torch.equal(out.view(torch.int32), ref.view(torch.int32))
    return out


def test_noalloc_matches_row_split_twice(sporder, ctx):
    """First call: 8000 rows with seven hub rows of 513 to 7000 nonzeros at
    N = 128; second call: a smaller matrix (3000 rows, two hubs) at N = 64."""
    print("[noalloc] n=8000 N=128 hubs", flush=True)
    big = hub_csr(8000, 9, {3: 7000, 77: 600, 4000: 7000, 4001: 513,
                            5000: 1025, 6001: 2048, 7999: 5000}, 61)
    assert (np.diff(big[0]) > 512).sum() == 7
    check_case(sporder, ctx, *big, N=128, seed=1)
    print("[noalloc] n=3000 N=64 hubs", flush=True)
    small = hub_csr(3000, 5, {10: 900, 2999: 1600}, 62)
    assert (np.diff(small[0]) > 512).sum() == 2
    check_case(sporder, ctx, *small, N=64, seed=2)


def test_noalloc_no_long_rows_and_scalar_width(sporder, ctx):
    """No long rows at N = 32 (no segments), and N = 30 (the scalar kernel)."""
    print("[noalloc] plain rows N=32, N=30", flush=True)
    plain = hub_csr(5000, 12, {}, 63)
    check_case(sporder, ctx, *plain, N=32, seed=3)
    check_case(sporder, ctx, *plain, N=30, seed=4)


def test_noalloc_rejects_oversized_scratch(sporder, ctx):
    """2048 rows of 1100 nonzeros at N = 4096: 6144 segment partial rows of
    16 KiB need 96 MiB, more than the 64 MiB array: ValueError, C untouched;
    a following call of normal size still matches."""
    print("[noalloc] oversized rejection", flush=True)
    n = 2048
    rng = np.random.default_rng(64)
    ind_h = np.sort(np.stack([rng.choice(n, 1100, replace=False) for _ in range(n)]),
                    axis=1).reshape(-1).astype(np.int32)
    ptr_h = (np.arange(n + 1) * 1100).astype(np.int32)
    val_h = rng.uniform(-1, 1, ind_h.size).astype(np.float32)
    ptr, ind, val = to_dev(ptr_h, ind_h, val_h)
    B = torch.ones((n, 4096), dtype=torch.float32, device="cuda:0")
    out = torch.zeros((n, 4096), dtype=torch.float32, device="cuda:0")
    with pytest.raises(ValueError, match="scratch"):
        sporder.spmm_csr_noalloc(ptr, ind, val, B, out=out, ctx=ctx)
    assert call_noalloc(sporder, ctx, ptr, ind, val, B, out) == _lib.SPMM_NOALLOC_TOO_LARGE
    assert int(torch.count_nonzero(out)) == 0
    del B, out
    check_case(sporder, ctx, ptr_h, ind_h, val_h, N=128, seed=5)


def test_noalloc_leaves_device_memory_unchanged(sporder):
    """On a fresh context (empty workspace), a call with long rows leaves the
    device's free memory as it was; sporder_spmm_csr on the same input and
    context then grows the workspace (n = 60000, 1.2 M nonzeros, N = 512:
    about 9 MiB of segment rows), which the same measurement sees, so the
    check can tell an allocation apart."""
    print("[noalloc] device memory unchanged on a fresh context", flush=True)
    ptr_h, ind_h, val_h = hub_csr(60000, 20, {7: 4000, 30000: 9000, 59999: 700}, 65)
    ptr, ind, val = to_dev(ptr_h, ind_h, val_h)
    n, N = ptr_h.shape[0] - 1, 512
    gen = torch.Generator(device="cuda:0").manual_seed(6)
    B = torch.randn((n, N), generator=gen, dtype=torch.float32, device="cuda:0")
    out = torch.zeros((n, N), dtype=torch.float32, device="cuda:0")
    ref = torch.zeros((n, N), dtype=torch.float32, device="cuda:0")
    fresh = sporder.Context()
    # One small call first, so that the context's stream and the kernels are
    # set up (the runtime may allocate for those on first use) before the
    # measured call.
    small = hub_csr(3000, 5, {10: 900}, 66)
    sptr, sind, sval = to_dev(*small)
    sB = torch.ones((3000, 64), dtype=torch.float32, device="cuda:0")
    sC = torch.empty((3000, 64), dtype=torch.float32, device="cuda:0")
    assert call_noalloc(sporder, fresh, sptr, sind, sval, sB, sC) == 0
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    assert call_noalloc(sporder, fresh, ptr, ind, val, B, out) == 0
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert free1 == free0, (free0, free1)
    _lib.load().sporder_spmm_csr(fresh.handle, n, ind.numel(), ptr.data_ptr(), ind.data_ptr(),
                                 val.data_ptr(), N, B.data_ptr(), ref.data_ptr(),
                                 _lib.SPMM_ROW_SPLIT, None)
    torch.cuda.synchronize()
    free2 = torch.cuda.mem_get_info()[0]
    assert free2 < free1, (free1, free2)
    assert torch.equal(out.view(torch.int32), ref.view(torch.int32))
