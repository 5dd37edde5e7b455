"""The reference's import paths (`mtc.*`) resolve to this package, and the legacy uniform
constructors `MTCMatrix.from_numpy` / `from_numpy_joint` write the reference's arena bytes.

CPU only: packing and byte layouts; the GPU side of these matrices is in
tests/test_gpu_dropin.py.
"""

import numpy as np
import pytest


def test_reference_import_paths_resolve_here():
    import mtc
    from mtc.core.allocation import META_BITS_PER_BLOCK, rd_allocate, rd_allocate_pair
    from mtc.core.permutation import PermutedQuadtreeRD, permuted_qt_dequant
    from mtc.core.quadtree import QuadtreeRD, qt_allocate, qt_dequant
    from mtc.core.types import PrecisionMode
    from mtc.kernels.gemm import MTCMatrix, mtc_gemm
    from mtc.kernels.reference import fp32_gemm_numpy, relative_frobenius_error

    import tensorpack_amd.core.allocation as TA
    import tensorpack_amd.core.permutation as TP
    import tensorpack_amd.core.quadtree as TQ
    import tensorpack_amd.kernels.gemm as TG
    assert MTCMatrix is TG.MTCMatrix and mtc_gemm is TG.mtc_gemm
    assert QuadtreeRD is TQ.QuadtreeRD and qt_dequant is TQ.qt_dequant and qt_allocate is TQ.qt_allocate
    assert PermutedQuadtreeRD is TP.PermutedQuadtreeRD and permuted_qt_dequant is TP.permuted_qt_dequant
    assert rd_allocate is TA.rd_allocate and rd_allocate_pair is TA.rd_allocate_pair
    assert META_BITS_PER_BLOCK == 40
    assert mtc.PrecisionMode is PrecisionMode and int(PrecisionMode.P16) == 16
    assert callable(fp32_gemm_numpy) and callable(relative_frobenius_error)


def test_packed_arena_accounting_through_mtc_paths():
    """Host half of the reference's tests/test_allocation.py:69-86 through the reference's
    import paths: the arena holds exactly the payload bits the allocator accounted for."""
    from mtc.core.allocation import rd_allocate_pair
    from mtc.kernels.gemm import MTCMatrix
    rng = np.random.RandomState(5)
    A = rng.randn(128, 96).astype(np.float32)
    B = rng.randn(96, 64).astype(np.float32)
    A[:, :32] *= 1e-4
    B[32:64] *= 20.0
    for budget in (2.6, 3.3, 5.2, 6.3, 9.0):
        a, b = rd_allocate_pair(A, B, budget)
        Am = MTCMatrix.from_allocation(A, a.modes, a.scales, 16)
        Bm = MTCMatrix.from_allocation(B, b.modes, b.scales, 16)
        assert Am.total_bytes_allocated * 8 == a.payload_bits
        assert Bm.total_bytes_allocated * 8 == b.payload_bits


def _block(m, Bs, i, j):
    return m[i * Bs:(i + 1) * Bs, j * Bs:(j + 1) * Bs]


def _codes_of(mm, i, j):
    """Signed row-major codes of block (i, j) read back from the arena bytes by hand:
    P8 int8, P16 little-endian int16, P4 two per byte low nibble first, P2 four per byte
    from bit 0 (mtc/kernels/gemm.py:29-117)."""
    Bs = mm.block_size
    P = int(mm.precisions[i, j])
    raw = mm.arena.raw_buffer[int(mm.offsets[i, j]): int(mm.offsets[i, j]) + P * Bs * Bs // 8]
    if P == 8:
        return raw.view(np.int8).astype(np.int64)
    if P == 16:
        return (raw[0::2].astype(np.int64) | (raw[1::2].astype(np.int64) << 8)).astype(np.uint16).view(np.int16).astype(np.int64)
    per = 8 // P
    out = []
    for byte in raw:
        for k in range(per):
            u = (int(byte) >> (P * k)) & ((1 << P) - 1)
            out.append(u - (1 << P) if u >= 1 << (P - 1) else u)
    return np.array(out, np.int64)


@pytest.mark.parametrize("mode,qmax,lo,hi", [(2, 1.0, -2, 1), (4, 7.0, -8, 7), (8, 127.0, -128, 127),
                                              (16, 32767.0, -32768, 32767)])
def test_from_numpy_fixed_mode_bytes(mode, qmax, lo, hi):
    from mtc.core.types import PrecisionMode
    from mtc.kernels.gemm import MTCMatrix
    rng = np.random.RandomState(mode)
    A = rng.randn(64, 48).astype(np.float32)
    A[:16, :16] = 0.0                               # a zero block: scale 1.0, all codes 0
    A[16:32, 16:32] *= 1e-9                         # max below 1e-7: scale 1.0, codes round to 0
    Bs = 16
    m = MTCMatrix.from_numpy(A, block_size=Bs, precision_mode=PrecisionMode(mode))
    assert m.pointer_tensor is None and m.shape == (64, 48) and m.block_size == Bs
    assert (m.precisions == mode).all()
    pos = 0
    for i in range(4):
        for j in range(3):
            blk = _block(A, Bs, i, j)
            amax = float(np.abs(blk).max())
            sc = amax / qmax if amax > 1e-7 else 1.0
            assert m.scales[i, j] == np.float32(sc)
            inv = np.float32(1.0 / sc)
            want = np.clip(np.rint(blk * inv), lo, hi).astype(np.int64).ravel()
            assert np.array_equal(_codes_of(m, i, j), want), (i, j)
            if mode == 16:
                pos += pos % 2
            assert int(m.offsets[i, j]) == pos
            pos += mode * Bs * Bs // 8
    assert m.total_bytes_allocated == pos
    assert m.arena.capacity >= max(1 << 20, 64 * 48 * 2)
    assert not _codes_of(m, 0, 0).any() and not _codes_of(m, 1, 1).any()


def test_from_numpy_adaptive_mode_choice():
    """Epsilon rule (mtc/core/precision.py:58-74): the lowest of P2/P4/P8 with relative error
    <= epsilon, else P16 at scale 1.0 (which rounds the block to integers)."""
    from mtc.kernels.gemm import MTCMatrix
    Bs = 8
    A = np.zeros((32, 32), np.float32)
    A[0:8, 0:8] = 0.5                     # constant block: exact at P2 (code 1, scale 0.5)
    A[0:8, 8:16] = np.linspace(-7, 7, 64).reshape(8, 8).round()   # integer grid -7..7: exact at P4
    rng = np.random.RandomState(0)
    A[8:16, 0:8] = rng.randn(8, 8)        # gaussian: P8 at eps 0.05, P2/P4 fail it
    A[8:16, 8:16] = rng.randn(8, 8) * 1e3
    m = MTCMatrix.from_numpy(A, block_size=Bs, epsilon=0.05)
    assert m.precisions[0, 0] == 2 and m.scales[0, 0] == np.float32(0.5)
    assert m.precisions[0, 1] == 4 and m.scales[0, 1] == np.float32(1.0)
    assert m.precisions[1, 0] == 8
    assert m.precisions[2, 2] == 2 and m.scales[2, 2] == np.float32(1.0)    # zero block
    # eps = 0: only exact reconstructions pass, the gaussian blocks fall back to P16 @ 1.0
    m0 = MTCMatrix.from_numpy(A, block_size=Bs, epsilon=0.0)
    assert m0.precisions[1, 0] == 16 and m0.scales[1, 0] == np.float32(1.0)
    assert np.array_equal(_codes_of(m0, 1, 0), np.rint(A[8:16, 0:8]).astype(np.int64).ravel())
    assert m0.precisions[0, 0] == 2 and m0.precisions[0, 1] == 4


def test_from_numpy_joint_negotiation():
    """Joint negotiation (mtc/core/precision.py:77-140, gemm.py:330-430): every block takes the
    highest mode any of its interacting pairs needs; each pair's chosen modes meet the
    product-error bound and every cheaper pair in the (sum, max) order misses it."""
    from mtc.core.precision import quantize_and_dequantize_block
    from mtc.kernels.gemm import MTCMatrix
    rng = np.random.RandomState(3)
    Bs, M, K, N = 8, 16, 24, 16
    A = rng.randn(M, K).astype(np.float32)
    B = rng.randn(K, N).astype(np.float32)
    A[:8, :8] *= 1e-6
    eps = 0.05
    ma, mb = MTCMatrix.from_numpy_joint(A, B, block_size=Bs, target_epsilon=eps)
    modes = (2, 4, 8, 16)
    pairs = sorted(((a, b) for a in modes for b in modes), key=lambda p: (p[0] + p[1], max(p)))

    def err(blk, m):
        rec, _ = quantize_and_dequantize_block(blk, m)
        return float(np.linalg.norm(blk.astype(np.float32) - rec.astype(np.float32)))

    need_a = np.full((M // Bs, K // Bs), 2)
    need_b = np.full((K // Bs, N // Bs), 2)
    for k in range(K // Bs):
        for i in range(M // Bs):
            for j in range(N // Bs):
                a, b = _block(A, Bs, i, k), _block(B, Bs, k, j)
                na, nb = float(np.linalg.norm(a)), float(np.linalg.norm(b))
                allowed = eps / np.sqrt(K // Bs) * na * nb
                ok = [(pa, pb) for pa, pb in pairs
                      if err(a, pa) * nb + na * err(b, pb) + err(a, pa) * err(b, pb) <= allowed]
                pa, pb = ok[0] if ok else (16, 16)
                need_a[i, k] = max(need_a[i, k], pa)
                need_b[k, j] = max(need_b[k, j], pb)
    assert np.array_equal(ma.precisions, need_a) and np.array_equal(mb.precisions, need_b)
    # joint packing uses each block's own max-abs scale at its negotiated mode
    qmag = {2: 1.0, 4: 7.0, 8: 127.0, 16: 32767.0}
    for i in range(M // Bs):
        for k in range(K // Bs):
            amax = float(np.abs(_block(A, Bs, i, k)).max())
            assert ma.scales[i, k] == np.float32(amax / qmag[int(ma.precisions[i, k])])


def test_from_numpy_rejects_unsupported():
    from mtc.core.types import PrecisionMode
    from mtc.kernels.gemm import MTCMatrix
    A = np.ones((16, 16), np.float32)
    with pytest.raises(ValueError):
        MTCMatrix.from_numpy(A, block_size=16, precision_mode=PrecisionMode.P3)
    with pytest.raises(ValueError):
        MTCMatrix.from_numpy(A, block_size=2)
    with pytest.raises(AssertionError):
        MTCMatrix.from_numpy(np.ones((20, 16), np.float32), block_size=16)


def test_precision_module_has_the_reference_names():
    """mtc.core.precision exposes the reference's helpers with its signatures: the error norms in
    closed form, and the two-block negotiation returning (pA, pB, scale_a, scale_b)."""
    from mtc.core.precision import (compute_frobenius_error, compute_relative_error, negotiate_joint_precision,
                                    quantize_and_dequantize_block)
    from mtc.core.types import PrecisionMode
    a = np.array([[3.0, 0.0], [0.0, 4.0]], np.float32)
    b = np.zeros((2, 2), np.float32)
    assert compute_frobenius_error(a, b) == 5.0 and compute_relative_error(a, b) == 1.0
    assert compute_relative_error(b, a) == 0.0                      # a zero block has no relative error
    assert negotiate_joint_precision(a, b) == (PrecisionMode.P2, PrecisionMode.P2, 1.0, 1.0)
    rng = np.random.RandomState(3)
    A, B = rng.randn(16, 16).astype(np.float32), rng.randn(16, 16).astype(np.float32)
    pa, pb, sa, sb = negotiate_joint_precision(A, B, target_epsilon=0.05)
    # the bound the rule checks, from the returned modes: ea*|B| + |A|*eb + ea*eb <= eps*|A||B|
    ea = compute_frobenius_error(A, quantize_and_dequantize_block(A, int(pa))[0])
    eb = compute_frobenius_error(B, quantize_and_dequantize_block(B, int(pb))[0])
    nA, nB = np.linalg.norm(A), np.linalg.norm(B)
    assert ea * nB + nA * eb + ea * eb <= 0.05 * nA * nB
    assert sa == quantize_and_dequantize_block(A, int(pa))[1] and sb == quantize_and_dequantize_block(B, int(pb))[1]
    # every cheaper pair (by total bits) violates it
    for qa in (2, 4, 8, 16):
        for qb in (2, 4, 8, 16):
            if qa + qb < int(pa) + int(pb):
                fa = compute_frobenius_error(A, quantize_and_dequantize_block(A, qa)[0])
                fb = compute_frobenius_error(B, quantize_and_dequantize_block(B, qb)[0])
                assert fa * nB + nA * fb + fa * fb > 0.05 * nA * nB
