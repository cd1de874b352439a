"""The C99 contract program (tests/c/contract.c) linked against
libsporder_hip.so, run on the GPU: every built entry point called from C and
its result checked (the reference runs sporder/tests/smoke.c as a CTest,
sporder/CMakeLists.txt:69-82)."""

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent / "c" / "sporder_contract"


def test_c_contract_program():
    assert EXE.exists(), "build() compiles tests/c/sporder_contract"
    res = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=120)
    print(res.stdout[-4000:], res.stderr[-4000:], flush=True)
    assert res.returncode == 0, res.stderr
    assert res.stdout.rstrip().endswith("contract: OK")
    assert res.stdout.count("contract: ok:") >= 18
