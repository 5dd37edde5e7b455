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


def kind_grid_stream(S, K=512, N=64, seed=31, merge_kinds=False):
    """Panel stream of S x S leaves only, each leaf's code width picked at random from every
    width (about 1 in 8 leaves P0), with random codes and power-of-two scales: every (S, P)
    kind occurs in every unit, so every decode path of that leaf size runs."""
    from tensorpack_amd.packer import CODE_WIDTHS, pack_levels
    rng = np.random.RandomState(seed + S)
    g = (K // S, N // S)
    modes = np.array((0,) + tuple(CODE_WIDTHS))[rng.randint(0, len(CODE_WIDTHS) + 1, size=g)]
    leaf = np.ones(g, bool)
    scales = (2.0 ** rng.randint(-9, -2, size=g)).astype(np.float32)
    codes = lambda S_, P, ii, jj, sc: rng.randint(-(1 << (P - 1)), 1 << (P - 1), size=(ii.size, S_, S_))
    return pack_levels((K, N), (S,), {S: leaf}, {S: modes}, {S: scales}, codes, chunk_rows=K,
                       merge_kinds=merge_kinds)


def kind_mix_stream(K=4096, N=32, seed=24):
    """Panel stream of 4x4 leaves whose code width changes with the column group (random
    codes, power-of-two scales, 30 % P0): the 4 column groups of a decode block step
    through different kinds, so a block has more step records than the fixed area holds
    (kinds are stored at their own widths: no merging into wider kinds)."""
    from tensorpack_amd.packer import pack_levels
    rng = np.random.RandomState(seed)
    widths = np.array([2, 3, 4, 5, 6, 8, 16, 2])
    modes4 = np.broadcast_to(np.resize(widths, N // 4)[None, :], (K // 4, N // 4)).copy()
    modes4[rng.rand(K // 4, N // 4) < 0.3] = 0
    leaf4 = np.ones((K // 4, N // 4), bool)
    scales4 = (2.0 ** rng.randint(-8, 0, size=(K // 4, N // 4))).astype(np.float32)
    codes = lambda S, P, ii, jj, sc: rng.randint(-(1 << (P - 1)), 1 << (P - 1), size=(ii.size, S, S))
    return pack_levels((K, N), (4,), {4: leaf4}, {4: modes4}, {4: scales4}, codes, chunk_rows=K, merge_kinds=False)
