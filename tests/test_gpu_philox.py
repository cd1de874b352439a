"""The SpMM hook's generator, Philox4x32-10 (chunkedgreedy_amd/csrc/philox.hpp),
run on the GPU by tests/c/philox_probe against the known-answer vectors
published with the generator (Random123's kat_vectors: counters 0, all ones
and the pi digits, keys 0, all ones and the next pi digits)."""

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

PROBE = Path(__file__).resolve().parent / "c" / "philox_probe"

KAT = [
    "6627e8d5 e169c58d bc57ac4c 9b00dbd8",
    "408f276d 41c83b0e a20bc7c6 6d5451fd",
    "d16cfe09 94fdcceb 5001e420 24126ea1",
]


def test_philox_known_answers():
    assert PROBE.exists(), "tests/c/philox_probe missing: run __graft_entry__.build()"
    out = subprocess.run([str(PROBE)], capture_output=True, text=True, timeout=60, check=True)
    assert out.stdout.split("\n")[:3] == KAT
