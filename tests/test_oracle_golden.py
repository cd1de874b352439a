"""The oracle against known answers that do not come from the oracle:

* hand-worked space-saving cases (tests/golden/sketch_cases.json, written by
  tests/golden/make_golden.py from the reference's rules);
* the band-matrix known answer from the reference smoke matrix
  (sporder/tests/smoke.c:58-70, 113-115);
* weighted_index packing (sporder/src/common/weighted_index.h:15-27);
* the defaults bridge (sporder/src/sporder.cpp:147-161) as closed forms.
"""

import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from chunkedgreedy_amd import synth

GOLDEN = json.loads((Path(__file__).parent / "golden" / "sketch_cases.json").read_text())


def padded(expected, k):
    idx = [e[0] for e in expected] + [-1] * (k - len(expected))
    return idx


@pytest.mark.parametrize("case", GOLDEN["stream_cases"], ids=lambda c: c["name"])
def test_sketch_stream_cases(case):
    w = np.array(case["weights_bits"], np.uint32).view(np.float32)
    out = oracle.sketch_stream(case["m"], case["k"], case["keys"], w)
    idx, wt = oracle.unpack_table(out[None, :])
    k = case["k"]
    assert idx[0].tolist() == padded(case["expected"], k)
    exp_bits = case["expected_bits"] + [0] * (k - len(case["expected"]))
    assert wt[0].view(np.uint32).tolist() == exp_bits


@pytest.mark.parametrize("case", GOLDEN["csr_cases"], ids=lambda c: c["name"])
def test_csr_stream_cases(case):
    ptr = np.array(case["ptr"], np.int32)
    ind = np.array(case["ind"], np.int32)
    for chk in case["checks"]:
        t = oracle.chunk_similarity_top_k(ptr, ind, case["k"], chk["chunk"], case["oversampling"])
        idx, wt = oracle.unpack_table(t)
        r = chk["row"]
        assert idx[r].tolist() == padded(chk["expected"], case["k"]), chk
        exp_bits = chk["expected_bits"] + [0] * (case["k"] - len(chk["expected"]))
        assert wt[r].view(np.uint32).tolist() == exp_bits, chk


def test_band_known_answer():
    kat = GOLDEN["band_kat"]
    ptr, ind, _ = synth.band(kat["n"], kat["half_width"])
    t = oracle.chunk_similarity_top_k(ptr, ind, kat["k"], kat["n"], kat["oversampling"],
                                      is_symmetric=True)
    idx, wt = oracle.unpack_table(t)
    assert idx[kat["row"]].tolist() == kat["expected_idx"]
    assert wt[kat["row"]].view(np.uint32).tolist() == kat["expected_bits"]
    # The sequential sum differs from the correctly rounded 6/7.
    assert kat["expected_bits"][0] == 0x3F5B6DB8
    assert kat["fl_6_7_bits"] == 0x3F5B6DB7
    # smoke.c:113-115: row 0 has a valid best neighbour.
    assert 0 < idx[0, 0] < kat["n"]


def test_band_global_is_chunk_n():
    """chunk_size >= n reproduces the global sketch (one chunk)."""
    ptr, ind, _ = synth.band(300)
    a = oracle.chunk_similarity_top_k(ptr, ind, 8, 300, 4.0, is_symmetric=True)
    b = oracle.chunk_similarity_top_k(ptr, ind, 8, 10_000, 4.0, is_symmetric=True)
    assert np.array_equal(a, b)


def test_weighted_index_packing():
    idx = np.array([-1, 0, 5, 2**31 - 2], np.int32)
    w = np.array([0.0, 1.5, 0.25, 3.0], np.float32)
    t = oracle.pack_table(idx, w)
    assert t[0] == 0  # the zero entry reads as (-1, +0.0)
    assert t[1] == (np.uint64(0x3FC00000) << np.uint64(32)) | np.uint64(1)
    i2, w2 = oracle.unpack_table(t)
    assert np.array_equal(i2, idx) and np.array_equal(w2.view(np.uint32), w.view(np.uint32))


@pytest.mark.parametrize("n,nnz,k,ovs,chunk,expect", [
    (20_000, 200_000, 0, 0.0, 0, (16, 4.0, 1024, 64)),       # C1
    (1_048_576, 16_777_216, 0, 0.0, 0, (16, 4.0, 1024, 64)),  # C2
    (4_096_000, 28_518_400, 0, 0.0, 0, (16, 4.0, 1024, 64)),  # C4 (nnz/n = 6)
    (1000, 26_000, 0, 0.0, 0, (26, 4.0, 1024, 128)),          # C5-like (k = 26, m = 104)
    (10, 10_000, 0, 0.0, 0, (256, 4.0, 1024, 1024)),           # k capped at 256
    (100, 300, 24, 2.5, 77, (24, 2.5, 77, 64)),                # m = 60 -> 64
    (100, 300, 5, 3.5, 7, (5, 3.5, 7, 32)),                    # m = 17 -> 32
])
def test_defaults_closed_form(n, nnz, k, ovs, chunk, expect):
    assert oracle.csg_defaults(n, nnz, k, ovs, chunk) == expect


def test_oracle_rejects_like_reference():
    ptr, ind, _ = synth.band(50)
    with pytest.raises(ValueError):  # k * oversampling > 512
        oracle.chunk_similarity_top_k(ptr, ind, 200, 10, 4.0, is_symmetric=True)
    with pytest.raises(ValueError):  # oversampling < 1
        oracle.chunk_similarity_top_k(ptr, ind, 16, 10, 0.5, is_symmetric=True)
