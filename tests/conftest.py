"""Shared test setup: the `gpu` marker and import paths.

`-m "not gpu"` tests run on any host (oracle vs golden vectors and closed
forms, host logic, C-ABI exports).  `-m gpu` tests call libsporder_hip.so on a
ROCm GPU and compare with the oracle.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")


@pytest.fixture(scope="session")
def sporder():
    """The sporder API; fails (does not skip) when the library or GPU is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test selected but torch.cuda.is_available() is False")
    from chunkedgreedy_amd import sporder as sp

    return sp


@pytest.fixture(scope="session")
def dev():
    return "cuda:0"
