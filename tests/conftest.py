import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


def say(msg: str) -> None:
    """Print and flush a progress line (names the case before each GPU step)."""
    print(msg, flush=True)


@pytest.fixture
def rng():
    return np.random.default_rng(0x2F6E2B1)
