"""Host logic of the harness counterparts and the generators (CPU), and the
plugins end to end on the GPU."""

import numpy as np
import pytest
import scipy.sparse as sp

import oracle
from chunkedgreedy_amd import harness, synth


def test_row_perm_and_apply_row_perm():
    a = sp.random(50, 50, density=0.1, format="csr", random_state=1, dtype=np.float32)
    perm = np.random.default_rng(0).permutation(50)
    assert np.array_equal(harness.row_perm_from_order(perm, 50), perm)
    with pytest.raises(ValueError):
        harness.row_perm_from_order(perm[:-1], 50)
    b = harness.apply_row_perm(a, perm)
    assert np.allclose(b.toarray(), a.toarray()[perm][:, perm])


def test_spmm_registry():
    m = harness.SpMMMethod.create("hip-csr-spmm")
    assert m.name == "hip-csr-spmm" and m.tc_h == 0 and m.uses_feature_dim
    assert harness.SpMMMethod.create("hip-csr-spmm-merge").algo == "merge_path"
    with pytest.raises(ValueError):
        harness.SpMMMethod.create("cusparse-spmm")


@pytest.mark.parametrize("gen,sym", [(lambda: synth.config1(1), False),
                                     (lambda: synth.stencil7(6, 2), True),
                                     (lambda: synth.rmat(9, 8, 3), True),
                                     (lambda: synth.chung_lu(3000, 2.1, 25, 4), True)])
def test_generators_shape(gen, sym):
    ptr, ind, val = gen()
    n = ptr.shape[0] - 1
    assert ptr[0] == 0 and ptr[-1] == ind.shape[0] == val.shape[0]
    assert ind.min() >= 0 and ind.max() < n
    rows = np.repeat(np.arange(n), np.diff(ptr))
    key = rows.astype(np.int64) * n + ind
    assert np.all(np.diff(key) > 0)  # sorted, distinct per row
    assert synth.is_pattern_symmetric(ptr, ind) == sym


def test_config1_planted_structure():
    ptr, ind, val = synth.config1(1)
    assert ptr.shape[0] - 1 == 20_000 and ind.shape[0] == 200_000
    assert np.all(np.diff(ptr) == 10)
    assert val.min() >= -1.0 and val.max() < 1.0


def test_stencil_nnz_closed_form():
    g = 9
    ptr, _, val = synth.stencil7(g, 1)
    assert ptr[-1] == 7 * g**3 - 6 * g**2
    assert np.isclose(val.sum(), 6 * g**3 - (6 * g**3 - 6 * g**2))


@pytest.mark.gpu
def test_reorder_plugin_matches_oracle(sporder):
    ptr, ind, val = synth.config1(8)
    a = sp.csr_matrix((val, ind, ptr), shape=(20_000, 20_000))
    res = harness.reorder(a, {"k": 0, "oversampling": 0.0, "chunk_size": 0,
                              "auto_detect_symmetric": True})
    o, _ = oracle.chunk_similarity_greedy(ptr, ind, is_symmetric=False)
    assert np.array_equal(res.row_perm, o.astype(np.int64))
    assert res.reorder_time_ms > 0 and res.effective_params == {"is_symmetric": False}
    assert set(res.timing_breakdown) == {"csr2csc_ms", "similarity_ms", "chunk_greedy_ms"}


@pytest.mark.gpu
def test_cg_reorder_plugin_matches_oracle(sporder):
    ptr, ind, val = synth.config1(10)
    a = sp.csr_matrix((val, ind, ptr), shape=(20_000, 20_000))
    res = harness.REORDER_METHODS["sporder-cg"](a, {"k": 0, "oversampling": 0.0,
                                                   "chunk_size": 0,
                                                   "auto_detect_symmetric": True})
    o, _ = oracle.chunk_greedy(ptr, ind, is_symmetric=False)
    assert np.array_equal(res.row_perm, o.astype(np.int64))
    assert set(res.timing_breakdown) == {"csr2csc_ms", "similarity_ms", "chunk_greedy_ms"}


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["hip-csr-spmm", "hip-csr-spmm-merge"])
def test_spmm_plugin(sporder, name):
    ptr, ind, val = synth.config1(9)
    a = sp.csr_matrix((val, ind, ptr), shape=(20_000, 20_000))
    m = harness.SpMMMethod.create(name)
    m.build()
    prepared = m.prepare(a)
    B = harness.generate_dense(20_000, 32, device="cuda:0")
    out, ms = m.run(prepared, B)
    ref = a.astype(np.float64) @ B.cpu().numpy().astype(np.float64)
    assert np.abs(out.cpu().numpy() - ref).max() / np.abs(ref).max() < 1e-5
    assert ms > 0
    assert harness.time_run(m, prepared, B, warmup=2, iterations=3) > 0


@pytest.mark.gpu
def test_spmm_plugin_blocked_tiles(sporder):
    """prepare builds an SpMM plan: on a band every 64-row tile runs in 8-row
    blocks, and the plugin's C equals the oracle's stated fmaf order bit for
    bit at N = 128."""
    ptr, ind, _ = synth.band(4096, 8)
    val = np.random.default_rng(3).uniform(-1, 1, ind.shape[0]).astype(np.float32)
    a = sp.csr_matrix((val, ind, ptr), shape=(4096, 4096))
    m = harness.SpMMMethod.create("hip-csr-spmm")
    prepared = m.prepare(a)
    assert prepared[3].info["blocked_tiles"] == 64
    B = harness.generate_dense(4096, 128, device="cuda:0")
    out, ms = m.run(prepared, B)
    want = oracle.spmm_csr(ptr, ind, val, B.cpu().numpy())
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32)) and ms > 0


@pytest.mark.gpu
def test_reorder_to_perm_npz_and_csv_row(sporder, tmp_path):
    """The csg plugin's permutation flows into the reference formats: the
    .perm.npz round trip, and a CSV row whose structure metrics (computed on
    the GPU for P A P^T) equal the oracle's on scipy's A[p, :][:, p]."""
    import csv

    import torch

    from chunkedgreedy_amd import formats, quality

    ptr, ind, val = synth.config1(12)
    a = sp.csr_matrix((val, ind, ptr), shape=(20_000, 20_000))
    params = {"k": 0, "chunk_size": 0, "oversampling": 0, "auto_detect_symmetric": True}
    res = harness.reorder(a, params)
    path = formats.save_reorder_perm(tmp_path, "C1", "sporder-csg", params, res.row_perm)
    perm = formats.load_reorder_perm(path, 20_000)
    assert np.array_equal(perm, res.row_perm)
    dptr = torch.from_numpy(ptr).cuda()
    dind = torch.from_numpy(ind).cuda()
    m = quality.reorder_bench_metrics(dptr, dind, torch.from_numpy(perm.astype(np.int32)).cuda())
    b = a[perm, :][:, perm].tocsr()
    b.sort_indices()
    want = oracle.reorder_bench_metrics(b.indptr, b.indices)
    assert {k: m[k] for k in want} == pytest.approx(want)
    out = tmp_path / "reorder_bench.csv"
    formats.write_result_row(out, formats.reorder_result_row("C1", "sporder-csg", params, res, m))
    with out.open() as fh:
        row = next(csv.DictReader(fh))
    assert row["reorder_hash"] == "a609629886c6" and int(row["tc_num"]) == want["tc_num"]
