"""The HBM ceiling kernels (sporder_hbm_stream) through the C ABI: a copy
copies, a write writes 1.0f, a read leaves its sink alone, on buffers that
are not a multiple of a workgroup's 16 KiB span; and the rates of a 256 MiB
run are positive and below the 8 TB/s peak."""

import ctypes

import pytest
import torch

from chunkedgreedy_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nt", [0, 1])
@pytest.mark.parametrize("nbytes", [16, 16 * 1000 + 16, (1 << 20) + 48])
def test_stream_kernels_move_the_data(sporder, nt, nbytes):
    print(f"[hbm] nbytes={nbytes} nt={nt}", flush=True)
    ctx = sporder.Context()
    lib = _lib.load()
    n = nbytes // 4
    src = torch.arange(n + 4, dtype=torch.int32, device="cuda:0")
    dst = torch.full((n + 4,), -7, dtype=torch.int32, device="cuda:0")
    ms = ctypes.c_float()
    lib.sporder_hbm_stream(ctx.handle, _lib.STREAM_COPY, nt, dst.data_ptr(), src.data_ptr(),
                           nbytes, 2, ctypes.byref(ms))
    assert torch.equal(dst[:n], src[:n]) and bool((dst[n:] == -7).all())
    assert ms.value > 0
    lib.sporder_hbm_stream(ctx.handle, _lib.STREAM_WRITE, nt, dst.data_ptr(), None, nbytes, 1,
                           None)
    assert bool((dst[:n].view(torch.float32) == 1.0).all()) and bool((dst[n:] == -7).all())
    before = dst.clone()
    lib.sporder_hbm_stream(ctx.handle, _lib.STREAM_READ, nt, dst.data_ptr(), src.data_ptr(),
                           nbytes, 1, None)
    assert torch.equal(dst, before)


def test_stream_rates_below_peak(sporder):
    from chunkedgreedy_amd.hbm import hbm_ceiling

    print("[hbm] 256 MiB rates", flush=True)
    rates = hbm_ceiling(256 << 20, 3)
    print(rates, flush=True)
    for op in ("read", "write", "copy"):
        for key in ("gbs", "gbs_nt"):
            assert 0 < rates[op][key] < 8000.0 * 1.05, (op, key, rates[op][key])
