"""Shared pytest configuration.

Markers
  gpu: needs an MI355X (gfx950) and the built native library; deselect with
       -m "not gpu" on machines without a GPU.
"""

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: requires an MI355X GPU and the built gfx950 library")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture
def rng():
    return np.random.default_rng(42)
