"""Shared pytest setup: the `gpu` marker and the repository on sys.path."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libfe_paged.so")


@pytest.fixture
def rng():
    return np.random.default_rng(1234)
