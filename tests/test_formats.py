"""Harness formats: reorder hash, .perm.npz and the reorder-bench CSV."""

import csv

import numpy as np
import pytest

from chunkedgreedy_amd import formats
from chunkedgreedy_amd.harness import ReorderResult

PAPER_PARAMS = {"k": 0, "chunk_size": 0, "oversampling": 0, "auto_detect_symmetric": True}


def test_hashes_match_paper_config():
    # Golden hashes of the reference's paper configuration (configs/paper.yaml:6,12,15).
    assert formats.compute_reorder_hash("sporder-csg", PAPER_PARAMS) == "a609629886c6"
    assert formats.compute_reorder_hash("sporder-cg", PAPER_PARAMS) == "eefae4eb9269"
    assert formats.compute_reorder_hash("ORIGIN", {}) == "685c3b160263"
    # Integral floats canonicalise to ints; key order does not matter.
    p2 = {"auto_detect_symmetric": True, "oversampling": 0.0, "chunk_size": 0, "k": 0}
    assert formats.compute_reorder_hash("sporder-csg", p2) == "a609629886c6"
    assert formats.compute_reorder_hash("sporder-csg", PAPER_PARAMS, {"omp_threads": 8}) \
        != "a609629886c6"


def test_perm_npz_round_trip(tmp_path):
    perm = np.random.default_rng(0).permutation(1000)
    path = formats.save_reorder_perm(tmp_path, "m1", "sporder-csg", PAPER_PARAMS, perm,
                                     source="test")
    assert path == tmp_path / "sporder-csg" / "m1_a609629886c6.perm.npz"
    assert np.array_equal(formats.load_reorder_perm(path, 1000), perm)
    with np.load(path, allow_pickle=False) as z:
        assert set(z.files) == {"row_perm", "matrix", "reorder_method", "params_json",
                                "reorder_hash", "env_json", "created_at", "source"}
        assert str(z["reorder_hash"]) == "a609629886c6"
        assert z["row_perm"].dtype == np.int64
    with pytest.raises(ValueError):
        formats.save_reorder_perm(tmp_path, "m1", "sporder-csg", PAPER_PARAMS, [0, 0, 1])
    with pytest.raises(ValueError):
        formats.load_reorder_perm(path, 999)


def test_result_csv(tmp_path):
    res = ReorderResult(row_perm=np.arange(4), reorder_time_ms=1.5, prep_time_ms=0.25,
                        perm_trans_ms=0.1, timing_breakdown={"similarity_ms": 1.0},
                        effective_params={"is_symmetric": False})
    row = formats.reorder_result_row("m1", "sporder-csg", PAPER_PARAMS, res,
                                     {"bandwidth": 3, "profile": 7, "tc_h": 16, "tc_w": 8,
                                      "tc_num": 2, "tc_fill_rate": 0.5})
    out = tmp_path / "r.csv"
    formats.write_result_row(out, row)
    formats.write_result_row(out, row)
    with out.open() as fh:
        rows = list(csv.DictReader(fh))
    assert list(rows[0]) == formats.RESULT_COLUMNS and len(rows) == 2
    assert rows[0]["reorder_hash"] == "a609629886c6" and rows[0]["reorder_time_ms"] == "1.5000"
    bad = tmp_path / "bad.csv"
    bad.write_text("a,b\n1,2\n")
    with pytest.raises(ValueError):
        formats.write_result_row(bad, row)
