"""Seeded random shapes, budgets and leaf mixes through every GPU entry point, against the
oracle: W_hat bit-exact (dequant), fp32 decode within 1e-5, bf16 prefill within 2e-3 of the
fp64 product of bf16-rounded X, and grouped launches bit-identical to single calls."""

import numpy as np
import pytest

from oracle import mtc_oracle as O
from tensorpack_amd.core.permutation import PermutedQuadtreeRD
from tensorpack_amd.core.quadtree import QuadtreeRD
from tensorpack_amd.kernels.gemm import MTCMatrix, mtc_gemm, mtc_gemm_group

from conftest import outlier_matrix

pytestmark = pytest.mark.gpu

SEEDS = list(range(12))


def _case(seed):
    r = np.random.RandomState(1000 + seed)
    sizes = (32, 16, 8, 4) if r.rand() < 0.7 else (16, 8, 4)
    root = sizes[0]
    K = root * int(r.randint(1, 1024 // root + 1))
    N = 32 * int(r.randint(1, 17))
    N = -(-N // root) * root
    perm = bool(r.rand() < 0.5)
    budget = float(np.round(r.uniform(2.0 if not perm else 2.2, 10.0), 3))
    return sizes, K, N, perm, budget, r


def _oracle_what(alloc, W):
    if hasattr(alloc, "inner"):
        i = alloc.inner
        return O.permuted_qt_dequant(W, alloc.row_perm, alloc.col_perm, i.sizes, i.leaf, i.modes, i.scales)
    return O.qt_dequant(W, alloc.sizes, alloc.leaf, alloc.modes, alloc.scales)


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz_shapes_budgets_and_paths(gpu, seed):
    import torch
    sizes, K, N, perm, budget, r = _case(seed)
    print("fuzz", seed, sizes, K, N, perm, budget, flush=True)
    W = outlier_matrix(2000 + seed, K, N)
    h = np.exp(r.randn(K))
    a = (PermutedQuadtreeRD if perm else QuadtreeRD)(W, h, sizes).select(budget)
    m = MTCMatrix.from_quadtree(a, W)
    what = _oracle_what(a, W)
    got = m.to_array()
    assert np.array_equal(got.view(np.uint32), what.view(np.uint32))
    M1 = int(r.randint(1, 17))
    X1 = r.randn(M1, K).astype(np.float32)
    Y1 = mtc_gemm(torch.from_numpy(X1).to(gpu), m).cpu().numpy()
    assert O.relative_frobenius_error(O.qt_gemm_f64(X1, what), Y1) <= 1e-5
    M2 = int(r.randint(17, 400))
    X2 = r.randn(M2, K).astype(np.float32)
    Y2 = mtc_gemm(torch.from_numpy(X2).to(gpu), m).cpu().numpy()
    assert O.relative_frobenius_error(O.qt_gemm_f64(O.bf16_round(X2), what), Y2) <= 2e-3
    # the same matrix twice in a group: each output equals the single call
    for X in (X1, X2):
        Xd = torch.from_numpy(X).to(gpu)
        ys = mtc_gemm_group(Xd, [m, m])
        single = mtc_gemm(Xd, m)
        assert all(torch.equal(y, single) for y in ys)
