"""The forms of the space-saving update at capacity 128 (add() item by item,
the compiled feed_generic(), the GCN-assembly feed4(), and the probe's own
rank-per-slot alternative) leave the same slots, bit for bit, on streams
dominated by evictions and by hits, for one wave and for many
(tests/c/sketch_probe, built by build()).  The probe also prints each form's
cost (kernel time, whole-GPU items/s, cycles per item of a wave)."""

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

PROBE = Path(__file__).resolve().parent / "c" / "sketch_probe"


@pytest.mark.parametrize("args", [
    ("16384", "1"),                               # half hot, half cold: mostly evictions
    ("8192", "1", "100", "100", "0.9"),           # mostly hits
    ("4096", "1", "60", "60", "0.5"),             # 120 keys: fills and hits, no eviction
    ("2048", "512"),                              # many waves
])
def test_sketch_forms_agree(args):
    assert PROBE.exists(), "tests/c/sketch_probe missing: run __graft_entry__.build()"
    print(f"[sketch_probe] {' '.join(args)}", flush=True)
    out = subprocess.run([str(PROBE), *args], capture_output=True, text=True, timeout=120)
    print(out.stdout, flush=True)
    assert out.returncode == 0, out.stdout + out.stderr
    agree = [line for line in out.stdout.splitlines() if "equals_form0" in line]
    assert agree == ["form=1 equals_form0=yes", "form=2 equals_form0=yes",
                     "form=3 equals_form0=yes", "form=4 equals_form0=yes"]


ISSUE = Path(__file__).resolve().parent / "c" / "issue_probe"


def test_issue_probe_runs():
    """tests/c/issue_probe: one wave's cost per instruction group (the cost
    model of the single-row sketch chain).  Checks that every group ran and
    that the costs it prints are positive; the figures are printed."""
    assert ISSUE.exists(), "tests/c/issue_probe missing: run __graft_entry__.build()"
    print("[issue_probe] 2000", flush=True)
    out = subprocess.run([str(ISSUE), "2000"], capture_output=True, text=True, timeout=120)
    print(out.stdout, flush=True)
    assert out.returncode == 0, out.stdout + out.stderr
    rows = [line.split() for line in out.stdout.splitlines() if line.startswith("group=")]
    assert len(rows) == 12
    for row in rows:
        assert float(row[2].split("=")[1]) > 0.0, row
