import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libmtc_hip.so")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def has_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    if not has_gpu():
        pytest.skip("no GPU")
    import torch
    return torch.device("cuda", 0)


def outlier_matrix(seed=0, n=128, m=None):
    """Small weights with 1% large outliers (tests/test_quadtree.py:13-18 recipe)."""
    m = n if m is None else m
    rng = np.random.RandomState(seed)
    W = (rng.randn(n, m) * 0.05).astype(np.float32)
    mask = rng.rand(n, m) < 0.01
    W[mask] = rng.uniform(-25, 25, size=mask.sum())
    return W
