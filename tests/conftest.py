import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "mamba-ascendc_amd")
for path in (ROOT, PKG_DIR):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(autouse=True)
def fixed_seed():
    """Deterministic torch RNG for every test (tests/mamba2/conftest.py:8-14)."""
    torch.manual_seed(42)
    yield


def gpu_available() -> bool:
    return torch.cuda.is_available()
