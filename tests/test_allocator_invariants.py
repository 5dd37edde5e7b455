"""Allocator invariants, mirroring the reference's own tests:
tests/test_quadtree.py:24-63, tests/test_permutation.py:23-61,
tests/test_allocation.py:17-66 -- plus checks of the scale search itself."""

import math

import numpy as np
import pytest

from tensorpack_amd.core import allocation as A
from tensorpack_amd.core.allocation import (META_BITS_PER_BLOCK, QRANGE, rd_allocate, rd_candidates,
                                            round_bf16)
from tensorpack_amd.core.permutation import PermutedQuadtreeRD, channel_orders, index_bits, permuted_qt_dequant
from tensorpack_amd.core.quadtree import QuadtreeRD, qt_allocate, qt_dequant

from conftest import outlier_matrix


def _rel(ref, pred):
    return float(np.linalg.norm(ref - pred) / np.linalg.norm(ref))


# ---------------- mode lattice ----------------
def test_code_ranges_and_grids():
    assert QRANGE == {2: (-2, 1), 3: (-4, 3), 4: (-8, 7), 5: (-16, 15), 6: (-32, 31), 8: (-128, 127),
                      16: (-32768, 32767)}
    sizes = {m: len(a) for m, a in A._ALPHAS.items()}
    assert sizes == {2: 33, 3: 29, 4: 25, 5: 21, 6: 17, 8: 9, 16: 1}
    for m, a in A._ALPHAS.items():
        assert a[-1] == 1.0
        if len(a) > 1:
            assert np.allclose(np.diff(a), 0.025)
    assert A.SCALE_FORMAT_META_BITS == {"fp32": 40, "bf16": 24} and META_BITS_PER_BLOCK == 40


# ---------------- bf16 scale rounding (allocation.py:97-103) ----------------
def _round_sig8_ref(x):
    if x == 0.0:
        return x
    m, e = math.frexp(x)
    return math.ldexp(round(m * 256.0) / 256.0, e)


def test_round_bf16_matches_frexp_formulation():
    rng = np.random.RandomState(0)
    x = np.concatenate([rng.randn(4000) * 10.0 ** rng.uniform(-30, 30, 4000),
                        # exact ties: 8 significant bits + a half ulp, both signs
                        np.array([(257 + 2 * k) / 512.0 * 2.0 ** e * sg for k in range(60)
                                  for e in (-5, 0, 7) for sg in (1, -1)])]).astype(np.float32)
    got = round_bf16(x)
    want = np.array([_round_sig8_ref(float(v)) for v in x], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # ties go to even: 1 + 1/256 + 1/512 -> 1 + 2/256 ; 1 + 1/512 -> 1.0
    assert round_bf16(np.array([1 + 3 / 512.0], np.float32))[0] == np.float32(1 + 2 / 256.0)
    assert round_bf16(np.array([1 + 1 / 512.0], np.float32))[0] == np.float32(1.0)


# ---------------- scale search vs a scalar restatement (allocation.py:106-136) ----------------
def _search_ref(block, h, mode, bf16):
    lo, hi = QRANGE[mode]
    qmag = float(max(-lo, hi))
    amax = np.float32(np.abs(block).max())
    amax = np.float32(1.0) if amax < 1e-30 else amax
    alphas = A._ALPHAS[mode].astype(np.float32)
    signs = [np.float32(1.0)] if mode == 16 else [np.float32(1.0), np.float32(-1.0)]
    bd, bs = np.inf, np.float32(0.0)
    for a in alphas:
        for sg in signs:
            s = np.float32(np.float64(np.float32(np.float32(sg * a) * amax)) / qmag)
            if bf16:
                s = np.float32(_round_sig8_ref(float(s)))
            inv = np.float32(1.0) / s
            d = 0.0
            for r in range(block.shape[0]):
                acc = np.float32(0.0)
                for c in range(block.shape[1]):
                    x = block[r, c]
                    q = np.float32(np.round(np.float32(x * inv)))
                    q = np.float32(lo) if q < lo else (np.float32(hi) if q > hi else q)
                    e = np.float32(x - np.float32(q * s))
                    acc = np.float32(acc + np.float32(e * e))
                d += float(h[r]) * float(acc)
            if d < bd:
                bd, bs = d, s
    return bd, bs


@pytest.mark.parametrize("mode", [2, 3, 5, 8, 16])
@pytest.mark.parametrize("bf16", [False, True])
def test_search_kernel_matches_scalar_restatement(mode, bf16):
    rng = np.random.RandomState(mode * 7 + bf16)
    W = (rng.standard_t(3, size=(8, 16)) * 0.3).astype(np.float32)
    W[:4, :4] = 0.0                                   # an all-zero block (amax floor)
    h = np.exp(rng.randn(8))
    hn = h / h.mean()
    c = rd_candidates(W, h, 4, (0, mode), "bf16" if bf16 else "fp32")
    blocks = A.to_blocks(W, 4)
    for i in range(2):
        for j in range(4):
            d_ref, s_ref = _search_ref(blocks[i, j], hn[4 * i:4 * i + 4], mode, bf16)
            assert c.S[1, i, j] == s_ref
            assert c.D[1, i, j] == d_ref


def test_p0_distortion_is_weighted_energy():
    rng = np.random.RandomState(3)
    W = rng.randn(16, 16).astype(np.float32)
    h = np.exp(rng.randn(16))
    c = rd_candidates(W, h, 8, (0, 4))
    hn = h / h.mean()
    e = (W.astype(np.float64) ** 2 * hn[:, None])
    want = e.reshape(2, 8, 2, 8).sum(axis=(1, 3))
    np.testing.assert_allclose(c.D[0], want, rtol=1e-12)


# ---------------- quadtree (tests/test_quadtree.py) ----------------
@pytest.mark.parametrize("budget", [2.0, 3.0, 4.5, 7.0])
def test_budget_respected_and_leaves_tile_exactly(budget):
    W = outlier_matrix()
    a = qt_allocate(W, budget, sizes=(32, 16, 8, 4))
    assert a.bits_per_element <= budget + 1e-9
    assert sum(a.leaf_area_fraction().values()) == pytest.approx(1.0)
    cover = np.zeros(W.shape, dtype=int)
    for s in a.sizes:
        cover += np.kron(a.leaf[s].astype(int), np.ones((s, s), dtype=int))
    assert (cover == 1).all()


def test_rebuild_is_exact():
    W = outlier_matrix(1)
    a = qt_allocate(W, 3.5)
    np.testing.assert_array_equal(qt_dequant(W, a.sizes, a.leaf, a.modes, a.scales), a.dequant)


def test_more_bits_less_error():
    W = outlier_matrix(2)
    qt = QuadtreeRD(W, None, (32, 16, 8, 4))
    errs = [_rel(W, qt.select(b).dequant) for b in (2.0, 3.0, 4.0, 6.0, 9.0)]
    assert all(e1 > e2 for e1, e2 in zip(errs, errs[1:]))


def test_quadtree_beats_fixed_tiles_on_localized_structure():
    W = outlier_matrix(3)
    fixed = rd_allocate(W, 3.0, None, 16, scale_format="bf16")
    tree = qt_allocate(W, 3.0, sizes=(32, 16, 8, 4))
    assert _rel(W, tree.dequant) < 0.7 * _rel(W, fixed.dequant)
    assert tree.leaf_area_fraction()[4] > 0.0


def test_quadtree_not_worse_on_homogeneous_data():
    W = np.random.RandomState(4).randn(128, 128).astype(np.float32)
    fixed = rd_allocate(W, 4.2, None, 16, scale_format="bf16")
    tree = qt_allocate(W, 4.2, sizes=(32, 16, 8))
    assert _rel(W, tree.dequant) <= 1.02 * _rel(W, fixed.dequant)


def test_scales_are_bf16_and_zero_off_leaves():
    W = outlier_matrix(5)
    a = qt_allocate(W, 3.0, sizes=(32, 16, 8, 4))
    for s in a.sizes:
        sc = a.scales[s]
        assert not np.any(sc.view(np.uint32) & 0xFFFF)
        assert np.all(sc[~a.leaf[s]] == 0) and np.all(sc[a.leaf[s] & (a.modes[s] == 0)] == 0)
        assert np.all(a.modes[s][~a.leaf[s]] == 0)


def test_infeasible_budget_raises():
    with pytest.raises(ValueError):
        QuadtreeRD(outlier_matrix(6), None, (32, 16)).select(0.01)
    with pytest.raises(ValueError):
        rd_allocate(outlier_matrix(6), 0.01)


# ---------------- permutation (tests/test_permutation.py) ----------------
def _row_scaled(K=256, N=256, seed=0):
    rng = np.random.RandomState(seed)
    W = (rng.randn(K, N) * np.exp(rng.randn(K, 1) * 1.0)).astype(np.float32)
    h = np.exp(rng.randn(K) * 0.5)
    return W, h


def test_orders_are_permutations():
    W, h = _row_scaled()
    pr, pc = channel_orders(W, h)
    assert np.array_equal(np.sort(pr), np.arange(W.shape[0]))
    assert np.array_equal(np.sort(pc), np.arange(W.shape[1]))
    keys = (h[:, None] * W.astype(np.float64) ** 2).sum(axis=1)
    assert np.all(np.diff(keys[pr]) >= 0)


@pytest.mark.parametrize("budget", [2.5, 4.25])
def test_budget_includes_index_bits(budget):
    W, h = _row_scaled()
    a = PermutedQuadtreeRD(W, h, (32, 16, 8)).select(budget)
    assert a.bits_per_element <= budget + 1e-9
    assert a.total_bits == a.inner.total_bits + index_bits(*W.shape, True, True)
    assert index_bits(256, 128, True, False) == 256 * 8


def test_rebuild_and_gather_scatter_inference_exact():
    W, h = _row_scaled()
    a = PermutedQuadtreeRD(W, h, (32, 16, 8)).select(3.0)
    inner = a.inner
    rebuilt = permuted_qt_dequant(W, a.row_perm, a.col_perm, inner.sizes, inner.leaf, inner.modes, inner.scales)
    np.testing.assert_array_equal(rebuilt, a.dequant)
    X = np.random.RandomState(1).randn(8, W.shape[0]).astype(np.float32)
    Y = np.empty((8, W.shape[1]), np.float32)
    Y[:, a.col_perm] = X[:, a.row_perm] @ inner.dequant
    ref = X @ a.dequant
    assert np.abs(Y - ref).max() <= 1e-6 * np.abs(ref).max()


def test_permutation_helps_on_shuffled_row_structure():
    W, h = _row_scaled()
    base = QuadtreeRD(W, h, (32, 16, 8, 4)).select(3.0)
    perm = PermutedQuadtreeRD(W, h, (32, 16, 8, 4)).select(3.0)

    def werr(Wq):
        return float((h[:, None] * (W - Wq) ** 2).sum())

    assert werr(perm.dequant) < 0.9 * werr(base.dequant)


# ---------------- uniform RD (tests/test_allocation.py) ----------------
@pytest.mark.parametrize("budget", [2.3, 3.0, 4.25, 6.0, 8.25])
def test_uniform_budget_is_respected(budget):
    W = np.random.RandomState(0).randn(128, 128).astype(np.float32)
    alloc = rd_allocate(W, budget)
    assert alloc.bits_per_element <= budget + 1e-9
    assert alloc.bits_per_element > budget - 16 * 256 / W.size


def test_uniform_error_decreases_with_budget():
    W = np.random.RandomState(1).randn(128, 128).astype(np.float32)
    errs = [_rel(W, rd_allocate(W, b).dequant) for b in (2.5, 3.5, 4.5, 6.5, 8.5)]
    assert all(e1 > e2 for e1, e2 in zip(errs, errs[1:]))


def test_uniform_homogeneous_data_matches_fixed_width():
    W = np.random.RandomState(2).randn(256, 256).astype(np.float32)
    budget = 4 + META_BITS_PER_BLOCK / 256.0
    adaptive = rd_allocate(W, budget)
    fixed = rd_allocate(W, budget, modes=(4,))
    assert _rel(W, adaptive.dequant) <= _rel(W, fixed.dequant) * 1.001


def test_importance_weighting_reduces_output_error():
    rng = np.random.RandomState(4)
    K, N, T = 256, 256, 128
    W = rng.randn(K, N).astype(np.float32)
    scale = np.ones(K)
    scale[rng.choice(K, 8, replace=False)] = 30.0
    X_cal = (rng.randn(T, K) * scale).astype(np.float32)
    X_test = (rng.randn(T, K) * scale).astype(np.float32)
    h = (X_cal ** 2).mean(axis=0)
    Y = X_test @ W
    assert _rel(Y, X_test @ rd_allocate(W, 3.0, h).dequant) < 0.8 * _rel(Y, X_test @ rd_allocate(W, 3.0, None).dequant)
