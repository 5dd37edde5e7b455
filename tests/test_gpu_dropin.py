"""The reference's own GPU-facing assertions, reached only through the reference's import
paths (`mtc.*`), on the HIP path.

- tests/test_allocation.py:69-86 (test_packed_kernel_matches_simulation): to_array is
  bit-exact to the allocator's dequant, mtc_gemm(A, B) within 1e-5 of the simulated product,
  arena bytes equal the accounted payload bits;
- tests/test_gemm.py:12-97: fixed P8 / P4, adaptive and joint uniform GEMMs within the
  reference's error bounds, plus to_array bit-exact to the arena's q * scale;
- a permuted quadtree matrix `mtc_gemm(X, W)` against the oracle's fp64 product.
"""

import numpy as np
import pytest

from mtc.core.allocation import rd_allocate_pair
from mtc.core.permutation import PermutedQuadtreeRD
from mtc.core.types import PrecisionMode
from mtc.kernels.gemm import MTCMatrix, mtc_gemm
from mtc.kernels.reference import fp32_gemm_numpy, relative_frobenius_error
from oracle import mtc_oracle as O

pytestmark = pytest.mark.gpu


def _rel(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / np.linalg.norm(a))


@pytest.mark.parametrize("budget", [2.6, 3.3, 5.2, 6.3, 9.0])
def test_packed_kernel_matches_simulation(gpu, budget):
    print("mtc path: packed kernel vs simulation, budget", budget, flush=True)
    rng = np.random.RandomState(5)
    A = rng.randn(128, 96).astype(np.float32)
    B = rng.randn(96, 64).astype(np.float32)
    A[:, :32] *= 1e-4
    B[32:64] *= 20.0
    a, b = rd_allocate_pair(A, B, budget)
    Am = MTCMatrix.from_allocation(A, a.modes, a.scales, 16)
    Bm = MTCMatrix.from_allocation(B, b.modes, b.scales, 16)
    np.testing.assert_allclose(Am.to_array(), a.dequant, rtol=0, atol=0)
    np.testing.assert_allclose(Bm.to_array(), b.dequant, rtol=0, atol=0)
    # the same W_hat from the oracle, bit for bit, and the product against the oracle's fp64 one
    A_hat, B_hat = O.uniform_to_array(A, a.modes, a.scales, 16), O.uniform_to_array(B, b.modes, b.scales, 16)
    assert np.array_equal(Am.to_array().view(np.uint32), A_hat.view(np.uint32))
    assert np.array_equal(Bm.to_array().view(np.uint32), B_hat.view(np.uint32))
    C_sim = a.dequant @ b.dequant
    assert _rel(C_sim, mtc_gemm(Am, Bm)) < 1e-5
    assert O.relative_frobenius_error(O.qt_gemm_f64(A_hat, B_hat), mtc_gemm(Am, Bm)) < 1e-5
    assert Am.total_bytes_allocated * 8 == a.payload_bits
    assert Bm.total_bytes_allocated * 8 == b.payload_bits


def _arena_hat(m):
    """q * scale per block, read from the arena bytes on the host (the reference's to_array,
    mtc/kernels/gemm.py:510-538)."""
    from mtc.kernels.gemm import arena_decode
    Bs = m.block_size
    out = np.zeros(m.shape, np.float32)
    for i in range(m.offsets.shape[0]):
        for j in range(m.offsets.shape[1]):
            P = int(m.precisions[i, j])
            o = int(m.offsets[i, j])
            q = arena_decode(m.arena.raw_buffer[o:o + P * Bs * Bs // 8][None], P, Bs * Bs)[0]
            out[i * Bs:(i + 1) * Bs, j * Bs:(j + 1) * Bs] = (q.astype(np.float32) * m.scales[i, j]).reshape(Bs, Bs)
    return out


@pytest.mark.parametrize("mode,bound", [(PrecisionMode.P8, 0.02), (PrecisionMode.P4, 0.25)])
def test_fixed_mode_gemm(gpu, mode, bound):
    print("mtc path: fixed", mode.name, flush=True)
    np.random.seed(42)
    N, Bs = 64, 16
    A = np.random.randn(N, N).astype(np.float32)
    B = np.random.randn(N, N).astype(np.float32)
    C_ref = fp32_gemm_numpy(A, B)
    ma = MTCMatrix.from_numpy(A, block_size=Bs, precision_mode=mode)
    mb = MTCMatrix.from_numpy(B, block_size=Bs, precision_mode=mode)
    assert np.array_equal(ma.to_array().view(np.uint32), _arena_hat(ma).view(np.uint32))
    assert np.array_equal(mb.to_array().view(np.uint32), _arena_hat(mb).view(np.uint32))
    C = mtc_gemm(ma, mb)
    assert relative_frobenius_error(C_ref, C) < bound
    assert _rel(_arena_hat(ma).astype(np.float64) @ _arena_hat(mb), C) < 1e-5


def test_adaptive_and_joint_gemm(gpu):
    print("mtc path: adaptive and joint", flush=True)
    np.random.seed(42)
    N, Bs = 64, 16
    A = np.random.randn(N, N).astype(np.float32)
    A[:32, :] *= 0.01
    B = np.random.randn(N, N).astype(np.float32)
    C_ref = fp32_gemm_numpy(A, B)
    ma = MTCMatrix.from_numpy(A, block_size=Bs, epsilon=0.05)
    mb = MTCMatrix.from_numpy(B, block_size=Bs, epsilon=0.05)
    C = mtc_gemm(ma, mb)
    assert relative_frobenius_error(C_ref, C) < 0.15
    assert _rel(_arena_hat(ma).astype(np.float64) @ _arena_hat(mb), C) < 1e-5
    np.random.seed(42)
    A = np.random.randn(N, N).astype(np.float32)
    B = np.random.randn(N, N).astype(np.float32)
    C_ref = fp32_gemm_numpy(A, B)
    ja, jb = MTCMatrix.from_numpy_joint(A, B, block_size=Bs, target_epsilon=0.05)
    Cj = mtc_gemm(ja, jb)
    assert relative_frobenius_error(C_ref, Cj) < 0.15
    assert _rel(_arena_hat(ja).astype(np.float64) @ _arena_hat(jb), Cj) < 1e-5
    assert np.array_equal(jb.to_array().view(np.uint32), _arena_hat(jb).view(np.uint32))


def test_permuted_quadtree_dense_x(gpu):
    import torch
    print("mtc path: QT-P dense X", flush=True)
    rng = np.random.RandomState(7)
    K, N = 512, 384
    W = (rng.standard_t(4, size=(K, N)) * 0.02).astype(np.float32)
    h = np.exp(rng.randn(K))
    a = PermutedQuadtreeRD(W, h, (32, 16, 8, 4)).select(4.25)
    m = MTCMatrix.from_allocation(W, a)
    i = a.inner
    W_hat = O.permuted_qt_dequant(W, a.row_perm, a.col_perm, i.sizes, i.leaf, i.modes, i.scales)
    assert np.array_equal(m.to_array().view(np.uint32), W_hat.view(np.uint32))
    assert np.array_equal(a.dequant.view(np.uint32), W_hat.view(np.uint32))
    for M in (1, 7, 16, 300):
        X = rng.randn(M, K).astype(np.float32)
        Y = mtc_gemm(X, m)                                   # numpy in -> numpy out
        ref = O.qt_gemm_f64(X, W_hat)
        tol = 1e-5 if M <= 16 else None
        if tol is None:
            ref = O.qt_gemm_f64(O.bf16_round(X), W_hat)
            tol = 2e-3
        assert isinstance(Y, np.ndarray) and Y.shape == (M, N)
        assert O.relative_frobenius_error(ref, Y) < tol, M
        Yt = mtc_gemm(torch.from_numpy(X).cuda(), m)        # device in -> device out
        assert Yt.is_cuda and np.array_equal(Yt.cpu().numpy(), Y)
