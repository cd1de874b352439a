"""Host logic of the configuration sweep (no GPU calls)."""

from chunkedgreedy_amd import sweep


def test_spmm_bytes_matches_c2_figures():
    # C2: n = 2^20, nnz = 2^24; N = 128 -> 1,212,153,860 B, N = 32 -> 406,847,492 B.
    assert sweep.spmm_bytes(1 << 20, 1 << 24, 128) == 1_212_153_860
    assert sweep.spmm_bytes(1 << 20, 1 << 24, 32) == 406_847_492


def test_widths_cover_every_config():
    assert sweep.WIDTHS == {"C1": [32], "C2": [32, 128], "C3": [32, 64, 256],
                            "C4": [16, 32, 64, 128, 256], "C5": [128]}


def test_main_needs_a_gpu(monkeypatch):
    import torch

    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    assert sweep.main(["--cfg", "C1"]) == 1
