"""The cross-lane rules the host model of the chain walk assumes
(tests/c/chain_model.cpp), measured on the GPU by tests/c/lane_probe (built
by build()): a shuffle from an inactive source lane returns 0, readlane reads
an inactive lane's value, a ballot sees only the active lanes."""

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

PROBE = Path(__file__).resolve().parent / "c" / "lane_probe"


def test_lane_rules():
    assert PROBE.exists(), "tests/c/lane_probe missing: run __graft_entry__.build()"
    out = subprocess.run([str(PROBE)], capture_output=True, text=True, timeout=60, check=True)
    rows = {line.split()[0]: line.split()[1:] for line in out.stdout.splitlines()}
    assert rows["shfl_inactive_source"] == ["0"] * 32
    assert rows["shfl_full_mask"] == [str(l + 132) for l in range(32)]
    assert rows["readlane_inactive"] == ["140"] * 32
    assert rows["ballot_half"] == ["0xffffffff"]
