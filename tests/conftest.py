"""Test configuration: the ``gpu`` marker and shared fixtures.

Tests marked ``gpu`` need a ROCm GPU and run the HIP kernels; everything else runs
on the CPU (oracle checks, host logic, the C ABI's loading and argument checks).
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

os.environ.setdefault("DEFORMOPS_FALLBACK_WARNINGS", "1")


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and runs the HIP kernels")
    config.addinivalue_line("markers", "slow: full-size workloads")


def gpu_available() -> bool:
    return torch.cuda.is_available() and torch.version.hip is not None


@pytest.fixture
def device() -> torch.device:
    if not gpu_available():
        pytest.skip("no ROCm GPU")
    return torch.device("cuda")


@pytest.fixture(autouse=True)
def _seed() -> None:
    torch.manual_seed(1958)
