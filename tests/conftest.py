"""Shared pytest configuration: the ``gpu`` marker and device helpers."""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libnlearn_hip.so")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no HIP device is visible")
    from nlearn_amd import _lib

    _lib.load()
    return torch.device("cuda:0")


def rel_l2(a, b, floor=0.0):
    """||a - b|| / max(||b||, floor * sqrt(b.size)). The floor keeps the ratio
    meaningful when the exact answer is (close to) zero."""
    import numpy as np

    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = max(np.linalg.norm(b), floor * np.sqrt(max(b.size, 1)), 1e-300)
    return float(np.linalg.norm(a - b) / den)
