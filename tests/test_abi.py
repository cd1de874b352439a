"""The C ABI: libsporder_hip.so loads and exports every symbol include/sporder.h
declares; struct layouts seen by C match the ctypes mirrors; the header
compiles as C99 (the reference checks the same, sporder/tests/smoke.c:1-12,
CMakeLists.txt:76-78).  No GPU calls."""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from chunkedgreedy_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "sporder.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(sporder_[a-z_]+)\s*\(", text)))


def test_header_declares_reference_entry_points():
    names = set(declared_symbols())
    reference = {"sporder_context_create", "sporder_context_destroy",
                 "sporder_hierarchical_matching", "sporder_chunk_greedy",
                 "sporder_chunk_similarity_greedy", "sporder_reorder",
                 "sporder_count_pillars", "sporder_bench_cusparse_spmm",
                 "sporder_similarity_graph", "sporder_similarity_graph_exact"}
    assert reference <= names
    assert names == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (sporder_\w+)", out))
    assert exported == set(declared_symbols())


STRUCTS = {
    "sporder_csg_timing_t": _lib.CsgTiming,
    "sporder_csg_stats_t": _lib.CsgStats,
    "sporder_cg_timing_t": _lib.CgTiming,
    "sporder_cg_stats_t": _lib.CgStats,
    "sporder_sim_timing_t": _lib.SimTiming,
    "sporder_sim_stats_t": _lib.SimStats,
    "sporder_hm_timing_t": _lib.HmTiming,
    "sporder_hm_stats_t": _lib.HmStats,
    "sporder_options_t": _lib.Options,
    "sporder_spmm_plan_info_t": _lib.SpmmPlanInfo,
}


def test_header_compiles_as_c99_and_layouts_match(tmp_path):
    lines = ['#include "sporder.h"', "#include <stdio.h>", "#include <stddef.h>",
             "int main(void) {"]
    for cname, st in STRUCTS.items():
        lines.append(f'  printf("{cname} %zu\\n", sizeof({cname}));')
        for field, _ in st._fields_:
            lines.append(f'  printf("{cname}.{field} %zu\\n", offsetof({cname}, {field}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", f"-I{HEADER.parent}", str(src), "-o",
                    str(exe)], check=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True,
                                                      text=True, check=True).stdout.splitlines())
    for cname, st in STRUCTS.items():
        assert int(got[cname]) == ctypes.sizeof(st), cname
        for field, _ in st._fields_:
            assert int(got[f"{cname}.{field}"]) == getattr(st, field).offset, (cname, field)


def test_product_path_fails_loudly_without_gpu():
    import torch

    if torch.cuda.is_available():
        pytest.skip("host has a GPU")
    from chunkedgreedy_amd import sporder

    with pytest.raises(RuntimeError):
        sporder.Context()
