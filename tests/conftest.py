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


def signed_scale_levels(seed=7, K=256, N=128, sizes=(32, 16, 8, 4)):
    """A random quadtree-like cover (each 32 x 32 root tile one leaf size), random code
    widths (about 1 in 8 leaves P0), bf16 power-of-two scales of random sign, and codes a
    fixed function of the leaf. Returns the pack_levels arguments and W_hat computed from the
    grids directly (q * s + 0.0 per leaf, so a zero code under a negative scale is +0.0)."""
    from tensorpack_amd.packer import CODE_WIDTHS
    rng = np.random.RandomState(seed)
    leaf = {s: np.zeros((K // s, N // s), bool) for s in sizes}
    modes = {s: np.zeros((K // s, N // s), np.int64) for s in sizes}
    scales = {s: ((2.0 ** rng.randint(-9, -1, size=(K // s, N // s))) *
                  rng.choice([-1.0, 1.0], size=(K // s, N // s))).astype(np.float32) for s in sizes}
    widths = np.array((0,) + tuple(CODE_WIDTHS))
    for i in range(K // 32):
        for j in range(N // 32):
            s = int(rng.choice(sizes))
            r = 32 // s
            leaf[s][i * r:(i + 1) * r, j * r:(j + 1) * r] = True
            modes[s][i * r:(i + 1) * r, j * r:(j + 1) * r] = widths[rng.randint(0, len(widths), size=(r, r))]
    base = {s: rng.randint(0, 1 << 16, size=(K // s, N // s, s, s)) for s in sizes}
    codes = lambda S, P, ii, jj, sc: base[S][ii, jj] % (1 << P) - (1 << (P - 1))
    W_hat = np.zeros((K, N), np.float32)
    for s in sizes:
        for i, j in zip(*np.nonzero(leaf[s] & (modes[s] > 0))):
            P = int(modes[s][i, j])
            q = (base[s][i, j] % (1 << P) - (1 << (P - 1))).astype(np.float32)
            W_hat[i * s:(i + 1) * s, j * s:(j + 1) * s] = q * scales[s][i, j] + np.float32(0.0)
    return ((K, N), sizes, leaf, modes, scales, codes), W_hat


def largest_unit_stream(seed=5):
    """The largest unit the panel stream allows: 4096 rows x 32 columns of 4x4 leaves, every
    one at P16 (65536 payload dwords and 8192 leaf words in one unit), random codes and
    power-of-two scales. Returns the stream and W_hat computed from the codes directly."""
    from tensorpack_amd.packer import pack_levels
    K, N = 4096, 32
    rng = np.random.RandomState(seed)
    g = (K // 4, N // 4)
    codes4 = rng.randint(-(1 << 15), 1 << 15, size=g + (4, 4))
    scales4 = (2.0 ** rng.randint(-24, -14, size=g)).astype(np.float32)
    W_hat = (codes4.astype(np.float32) * scales4[:, :, None, None]).transpose(0, 2, 1, 3).reshape(K, N)
    ps = pack_levels((K, N), (4,), {4: np.ones(g, bool)}, {4: np.full(g, 16)}, {4: scales4},
                     lambda S, P, ii, jj, sc: codes4[ii, jj], chunk_rows=K)
    return ps, W_hat + np.float32(0.0)


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
