"""Shared pytest configuration.

* ``gpu`` marker: tests that need an MI355X (gfx950).  The CPU suite runs with
  ``-m "not gpu"``; GPU tests call the kernels through the C ABI.
* Autouse seeding of ``random``, numpy and torch with 42, as the reference's
  ``tests/conftest.py:12-19`` does.
"""

from __future__ import annotations

import random
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(autouse=True)
def _seed_everything() -> None:
    random.seed(42)
    np.random.seed(42)
    torch.manual_seed(42)


@pytest.fixture()
def cuda() -> torch.device:
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    return torch.device("cuda:0")
