"""pytest configuration: the `gpu` marker (tests that need an MI355X) and shared helpers."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X, gfx950) and the built HIP library")
    config.addinivalue_line("markers", "slow: long CPU test")


def same_bits(a, b) -> bool:
    a = np.ascontiguousarray(a, np.float32).view(np.uint32)
    b = np.ascontiguousarray(b, np.float32).view(np.uint32)
    return a.shape == b.shape and bool(np.array_equal(a, b))


@pytest.fixture
def rng():
    return np.random.default_rng(0)
