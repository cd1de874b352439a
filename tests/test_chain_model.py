"""Host model of the compact chain walk (tests/c/chain_model.cpp), lane by lane.

The model follows the wave's cross-lane rules: ballots see active lanes,
readlane ignores the execution mask, and a shuffle (ds_bpermute) from an
inactive source lane returns 0 (measured on MI355X).  With those rules:

- the kernel's walk, in the mode the kernel picks and in each mode forced,
  gives the oracle's permutation on the test matrices and on full C2, with no
  out-of-chunk write, no row visited twice and no LDS index outside its array;
- the same holds under the narrow launch's configuration: chunks whose
  in-chunk entries pass the 2048 staged ones walk 16-bit packed rows (the
  kernel's packing: table order, runs of equal weight sorted by index), and
  chunks with 8193..16,384 valid entries go to the second, packed launch;
  every walk mode (table reads; one-entry and read-ahead on 64-bit and on
  packed rows) and both launches are reached;
- a removed variant, whose visited test ran its shuffles only in the lanes
  holding a candidate (`cl >= 0 && !visited(cl)`), reads visited rows as free,
  revisits them and writes past its chunk (its walk loop had no bound): the
  GPU memory fault it caused.  With the mask ignored, the same walk gives the
  oracle's permutation, so the shuffle rule is the whole difference.
"""

import ctypes
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle
from chunkedgreedy_amd import synth

HERE = Path(__file__).resolve().parent


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    so = tmp_path_factory.mktemp("chain_model") / "chain_model.so"
    subprocess.run(["g++", "-std=c++17", "-O2", "-shared", "-fPIC", "-o", str(so),
                    str(HERE / "c" / "chain_model.cpp")], check=True)
    lib = ctypes.CDLL(str(so))
    P = ctypes.c_void_p
    lib.chain_model.argtypes = [ctypes.c_int32] * 3 + [P] + [ctypes.c_int32] * 4 + [P, P, P]
    lib.chain_model.restype = ctypes.c_int32

    def run(table, chunk, entry_cap, variant, inactive_zero=1, packed_cap=0, all_modes=False):
        table = np.ascontiguousarray(table, np.uint64)
        n, k = table.shape
        order = np.full(n, -1, np.int32)
        diag = np.zeros(10, np.int64)
        modes = np.zeros(6, np.int64)
        rc = lib.chain_model(n, k, chunk, table.ctypes.data, entry_cap, packed_cap, variant,
                             inactive_zero, order.ctypes.data, diag.ctypes.data,
                             modes.ctypes.data)
        keys = ("overrun", "revisit", "oob", "misread", "runaway", "steps",
                "asm_end", "asm_restart", "asm_long", "asm_ring")
        m = modes.tolist()
        return rc, order, dict(zip(keys, diag.tolist())), (m if all_modes else m[:3])

    return run


MATS = {
    "band1000": synth.band(1000)[:2],
    "C1": synth.config1(11)[:2],
    "planted64k": synth.planted(1 << 16, 1024, 16, 12)[:2],
    "stencil20": synth.stencil7(20, 13)[:2],
    "stencil20_ordered": synth.stencil7(20, 13, scramble=False)[:2],
    "rmat13": synth.rmat(13, 16, 14)[:2],
    "chunglu20k": synth.chung_lu(20000, 2.1, 25, 15)[:2],
}
CASES = [(16, 1024), (8, 256), (32, 4096)]


def table_and_order(ptr, ind, k, chunk, sym=None):
    if sym is None:
        sym = synth.is_pattern_symmetric(ptr, ind)
    table = oracle.chunk_similarity_top_k(ptr, ind, k, chunk, 4.0, is_symmetric=sym)
    order, _ = oracle.greedy(table, chunk)
    return table, order


CLEAN = {"overrun": 0, "revisit": 0, "oob": 0, "misread": 0, "runaway": 0}


@pytest.mark.parametrize("name", sorted(MATS))
@pytest.mark.parametrize("k,chunk", CASES)
@pytest.mark.parametrize("entry_cap", [2048, 8192])
def test_kernel_walk_matches_oracle(model, name, k, chunk, entry_cap):
    table, want = table_and_order(*MATS[name], k, chunk)
    rc, order, diag, modes = model(table, chunk, entry_cap, 0)
    assert rc == 0
    assert {key: diag[key] for key in CLEAN} == CLEAN
    assert np.array_equal(order, want)
    # Every mode that applies to all chunks, forced, gives the same order.
    forced = [1, 2] if modes[0] == 0 else ([0] if modes[1] == modes[2] == 0 else [])
    for mode in forced:
        rc, order, diag, _ = model(table, chunk, entry_cap, mode + 1)
        assert rc == 0
        assert {key: diag[key] for key in CLEAN} == CLEAN
        assert np.array_equal(order, want), mode


@pytest.mark.parametrize("name", ["band1000", "C1", "planted64k", "rmat13"])
def test_removed_variant_writes_past_its_chunk(model, name):
    table, want = table_and_order(*MATS[name], 16, 1024)
    rc, order, diag, _ = model(table, 1024, 2048, 10, inactive_zero=1)
    assert rc == 0
    assert diag["misread"] > 0 and diag["revisit"] > 0 and diag["overrun"] > 0
    rc, order, diag, _ = model(table, 1024, 2048, 10, inactive_zero=0)
    assert rc == 0 and diag["overrun"] == 0 and diag["revisit"] == 0
    assert np.array_equal(order, want)


def test_full_c2(model):
    """Full C2 (csg defaults): the kernel's walk (the one-entry mode on every
    chunk) equals the oracle; the removed variant writes 1.9 M positions past
    its chunks."""
    ptr, ind = synth.config2()[:2]
    table, want = table_and_order(ptr, ind, 16, 1024, sym=False)  # as the bench line runs it
    rc, order, diag, modes = model(table, 1024, 2048, 0)
    assert rc == 0 and modes == [0, 1024, 0]
    assert {key: diag[key] for key in CLEAN} == CLEAN
    assert np.array_equal(order, want)
    rc, order, diag, _ = model(table, 1024, 2048, 10, inactive_zero=1)
    assert diag["overrun"] > 1_000_000 and diag["runaway"] > 0


# The host's packed capacity for the narrow launch (csg.hip: rows_max * k
# capped at kPackedCap = 16384, k <= kPackedMaxK = 32, no statistics).
def host_packed_cap(n, k, chunk):
    return min(min(chunk, n) * k, 16384) if k <= 32 else 0


@pytest.mark.parametrize("name", sorted(MATS))
@pytest.mark.parametrize("k,chunk", CASES)
def test_packed_walks_match_oracle(model, name, k, chunk):
    """The narrow launch's configuration (2048 staged entries, packed rows
    past that, the packed launch for slices of 8193..16,384 valid entries):
    every chunk, staged, packed or read from the table, gives the oracle's
    order in the mode the kernel picks and in each mode forced."""
    table, want = table_and_order(*MATS[name], k, chunk)
    pc = host_packed_cap(*table.shape, chunk)
    rc, order, diag, modes = model(table, chunk, 2048, 0, packed_cap=pc, all_modes=True)
    assert rc == 0
    assert {key: diag[key] for key in CLEAN} == CLEAN
    assert np.array_equal(order, want)
    forced = [1, 2] if modes[0] == 0 else ([0] if modes[1] == modes[2] == 0 else [])
    for mode in forced:
        rc, order, diag, _ = model(table, chunk, 2048, mode + 1, packed_cap=pc)
        assert rc == 0
        assert {key: diag[key] for key in CLEAN} == CLEAN
        assert np.array_equal(order, want), mode


def test_packed_modes_and_second_launch_are_exercised(model):
    """The matrices above reach both packed walk modes and both launches;
    a grid-ordered stencil (C4n's structure: every slice between 8192 and
    16,384 valid entries) runs all its chunks in the packed launch."""
    seen = np.zeros(6, np.int64)
    for name in sorted(MATS):
        for k, chunk in CASES:
            table, _ = table_and_order(*MATS[name], k, chunk)
            pc = host_packed_cap(*table.shape, chunk)
            rc, _, _, modes = model(table, chunk, 2048, 0, packed_cap=pc, all_modes=True)
            assert rc == 0
            seen += np.array(modes)
    assert seen[4] > 0 and seen[5] > 0, seen.tolist()  # packed read-ahead walks, second launch
    # Twin rows (rows 2i and 2i + 1 hold the same two columns): every row has
    # exactly one in-chunk entry, 4096 per 4096-row chunk, past the 2048
    # staged entries: the packed one-entry walk.
    n = 8192
    ptr = np.arange(0, 2 * n + 1, 2, dtype=np.int32)
    ind = np.repeat(np.arange(0, n, 2, dtype=np.int32), 2)
    ind = np.stack([ind, ind + 1], axis=1).reshape(-1).astype(np.int32)
    table, want = table_and_order(ptr, ind, 8, 4096)
    rc, order, diag, modes = model(table, 4096, 2048, 0, packed_cap=host_packed_cap(n, 8, 4096),
                                   all_modes=True)
    assert rc == 0 and {key: diag[key] for key in CLEAN} == CLEAN
    assert np.array_equal(order, want)
    assert modes[3] == 2, modes
    ptr, ind = synth.stencil7(24, 13, scramble=False)[:2]
    table, want = table_and_order(ptr, ind, 16, 1024)
    rc, order, diag, modes = model(table, 1024, 2048, 0, packed_cap=16384, all_modes=True)
    assert rc == 0 and {key: diag[key] for key in CLEAN} == CLEAN
    assert np.array_equal(order, want)
    chunks = -(-table.shape[0] // 1024)
    assert modes[3] + modes[4] == chunks and modes[5] >= chunks - 1, modes


def test_assembly_step_exits(model):
    """The read-ahead steps the kernel runs in assembly (chunks of at most 64
    bitmap words) hand a step back at a row of more than 64 in-chunk entries,
    at a row with no free entry and when the position ring is full; the model
    takes each of those returns and still gives the oracle's order.  Rows of
    about 70 and 40 in-chunk entries in one chunk (synth.dense_groups, k = 96,
    the 8192-entry staging of at most two chunks per CU); C1 at the same
    staging fills the ring."""
    ptr, ind, _ = synth.dense_groups()
    table, want = table_and_order(ptr, ind, 96, 1024)
    rc, order, diag, modes = model(table, 1024, 8192, 0)
    assert rc == 0 and {key: diag[key] for key in CLEAN} == CLEAN
    assert np.array_equal(order, want)
    assert modes[2] == 8, modes
    assert diag["asm_long"] > 0 and diag["asm_restart"] > 0, diag
    table, want = table_and_order(*MATS["C1"], 16, 1024)
    rc, order, diag, _ = model(table, 1024, 8192, 0)
    assert rc == 0 and {key: diag[key] for key in CLEAN} == CLEAN
    assert np.array_equal(order, want)
    assert diag["asm_ring"] > 0, diag
