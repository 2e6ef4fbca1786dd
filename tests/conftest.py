"""Shared pytest setup.

Markers: ``gpu`` tests need a ROCm GPU and the built libqmoe.so; everything
else runs on the CPU.  The repository root goes on sys.path so tests can
import ``titan_amd`` and the oracle (``oracle/oracle.py``).
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
if str(ROOT / "oracle") not in sys.path:
    sys.path.insert(0, str(ROOT / "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built libqmoe.so")
    config.addinivalue_line("markers", "slow: long-running")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from titan_amd import _lib

    _lib.load()  # a GPU test without the native library is a failure, not a skip
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.build()
    return oracle
