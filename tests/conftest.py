"""Shared test configuration.

Tests marked ``gpu`` need an MI355X (run with ``-m gpu``); everything else runs
on the CPU.  The repository root is put on sys.path so ``oracle`` and
``cacheslide_amd`` import without installation.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X)")


@pytest.fixture
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)
