import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through librq on cuda:0)")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    return torch.device("cuda", 0)


def norm_err(y, r):
    """max|y - r| / max|r| -- the gate metric for every fused matmul."""
    import numpy as np

    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    denom = float(np.max(np.abs(r))) if r.size else 0.0
    if denom == 0.0:
        return float(np.max(np.abs(y - r))) if r.size else 0.0
    return float(np.max(np.abs(y - r)) / denom)
