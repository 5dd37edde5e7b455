"""Tile stream (prefill layout): decodes to bf16(W_hat) exactly, keeps its
layout invariants (class-sorted cells, 16-byte aligned payload, every cell
position once per step), and codes every width class."""

import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

from oracle import mtc_oracle as O
from tensorpack_amd.core.allocation import rd_allocate
from tensorpack_amd.core.permutation import PermutedQuadtreeRD
from tensorpack_amd.core.quadtree import QuadtreeRD
from tensorpack_amd.kernels.gemm import MTCMatrix
from tensorpack_amd.tilestream import CELLS, CLS_DWORDS, CLS_Z, decode_tiles

from conftest import outlier_matrix


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _want(alloc, W):
    if hasattr(alloc, "inner"):
        i = alloc.inner
        w = O.permuted_qt_dequant(W, alloc.row_perm, alloc.col_perm, i.sizes, i.leaf, i.modes, i.scales)
    else:
        w = O.qt_dequant(W, alloc.sizes, alloc.leaf, alloc.modes, alloc.scales)
    return O.bf16_round(w) + np.float32(0.0)


@pytest.mark.parametrize("cls,budget,K,N", [(QuadtreeRD, 2.2, 128, 96), (QuadtreeRD, 4.5, 192, 320),
                                            (QuadtreeRD, 15.0, 64, 64), (PermutedQuadtreeRD, 3.1, 256, 288),
                                            (QuadtreeRD, 5.0, 96, 64)])
def test_tiles_decode_to_bf16_w_hat(cls, budget, K, N):
    W = outlier_matrix(int(budget * 7), K, N)
    a = cls(W, np.exp(np.random.RandomState(2).randn(K)), (32, 16, 8, 4)).select(budget)
    ts = MTCMatrix.from_quadtree(a, W).tile_stream()
    assert np.array_equal(_bits(decode_tiles(ts)), _bits(_want(a, W)))


def test_tile_layout_invariants():
    W = outlier_matrix(4, 192, 320)
    a = QuadtreeRD(W, None, (32, 16, 8, 4)).select(6.0)
    ts = MTCMatrix.from_quadtree(a, W).tile_stream()
    assert ts.n_ksteps == 3 and ts.n_col_tiles == 2
    assert np.all(ts.step_off % 4 == 0)
    for step in range(ts.n_steps):
        c = ts.cells[step * CELLS:(step + 1) * CELLS, 0].astype(np.int64)
        off, cls, pos = c & 0x3FFF, (c >> 14) & 3, c >> 16
        assert sorted(pos.tolist()) == list(range(CELLS))            # every cell once
        assert np.all(np.diff(cls * CELLS + pos) > 0)                 # class-sorted, then position
        size = CLS_DWORDS[cls]
        assert np.array_equal(off, np.concatenate([[0], np.cumsum(size)[:-1]]))
        assert ts.step_off[step + 1] - ts.step_off[step] == size.sum()
    # columns beyond N (second column tile holds 64 of 256) are zero cells
    last = ts.cells[(ts.n_steps - 1) * CELLS:, 0].astype(np.int64)
    beyond = (last >> 16) >= (320 - 256) // 4 * 8
    assert np.all(((last >> 14) & 3)[beyond] == CLS_Z)


def test_all_width_classes_present_and_fp32_scales():
    rng = np.random.RandomState(8)
    W = rng.randn(256, 128).astype(np.float32)
    al = rd_allocate(W, 9.0, None, 32)
    m = MTCMatrix.from_allocation(W, al.modes, al.scales, 32)
    ts = m.tile_stream()
    assert ts.fp32_scales and ts.cells.shape[1] == 4
    assert np.array_equal(_bits(decode_tiles(ts)), _bits(O.bf16_round(al.dequant) + np.float32(0.0)))
    W2 = outlier_matrix(3, 128, 128)
    a = QuadtreeRD(W2, None, (32, 16, 8, 4)).select(5.0)
    ts2 = MTCMatrix.from_quadtree(a, W2).tile_stream()
    classes = set(((ts2.cells[:, 0] >> 14) & 3).tolist())
    assert classes == {0, 1, 2, 3}, classes
    assert np.array_equal(_bits(decode_tiles(ts2)), _bits(_want(a, W2)))


@settings(max_examples=12, deadline=None)
@given(seed=st.integers(0, 10 ** 6), budget=st.floats(1.8, 16.0), perm=st.booleans(),
       sizes=st.sampled_from([(32, 16, 8, 4), (16, 8, 4), (8, 4), (4,), (32,)]))
def test_fuzz_tiles(seed, budget, perm, sizes):
    rng = np.random.RandomState(seed)
    W = (rng.randn(64, 96) * 10.0 ** rng.uniform(-2, 1, size=(64, 1))).astype(np.float32)
    W[rng.rand(64, 96) < 0.03] = 20.0
    cls = PermutedQuadtreeRD if perm else QuadtreeRD
    try:
        a = cls(W, np.exp(rng.randn(64)), sizes).select(budget)
    except ValueError:
        return
    ts = MTCMatrix.from_quadtree(a, W).tile_stream()
    assert np.array_equal(_bits(decode_tiles(ts)), _bits(_want(a, W)))


@pytest.mark.parametrize("K,N,budget", [(256, 288, 3.1), (192, 160, 11.0), (64, 96, 2.0)])
def test_gathered_columns_for_permuted_matrices(K, N, budget):
    """A QT-P matrix packs its columns back in the original order: 8-word cells with a scale pair
    per column, no col_perm, the same bf16 W_hat; column j's scale words name the leaf of the
    permuted column the original column comes from. gather_cols=False keeps the permuted order."""
    from tensorpack_amd.tilestream import TILE_COLS, TILE_ROWS, pack_tiles
    W = outlier_matrix(int(budget * 3), K, N)
    a = PermutedQuadtreeRD(W, np.exp(np.random.RandomState(6).randn(K)), (32, 16, 8, 4)).select(budget)
    m = MTCMatrix.from_quadtree(a, W)
    ts = m.tile_stream()
    assert ts.cols_gathered and ts.col_perm is None and ts.row_perm is not None and ts.cells.shape[1] == 8
    assert not ts.cells[:, 5:].any()
    assert np.array_equal(_bits(decode_tiles(ts)), _bits(_want(a, W)))
    # scale words against the allocation: original column n is permuted column inv[n]
    i = a.inner
    inv = np.argsort(a.col_perm)
    S_el = np.zeros((K, N), np.float32)
    for S in i.sizes:
        L = np.asarray(i.leaf[S], bool)
        sc = np.where(L, np.asarray(i.scales[S], np.float32), 0.0)
        S_el += np.kron(sc, np.ones((S, S), np.float32))
    S_orig = S_el[:, inv]                                     # permuted rows, original columns
    rng = np.random.RandomState(1)
    for idx in rng.choice(ts.cells.shape[0], 64, replace=False):
        step, w0 = idx // CELLS, int(ts.cells[idx, 0])
        ct, ks = divmod(step, ts.n_ksteps)
        pos = w0 >> 16
        r0, c0 = ks * TILE_ROWS + (pos & 7) * 8, ct * TILE_COLS + (pos >> 3) * 4
        if (w0 >> 14) & 3 == CLS_Z or r0 >= K or c0 >= N:
            continue
        for j in range(4):
            sw = int(ts.cells[idx, 1 + j])
            top = np.array([(sw & 0xFFFF) << 16], np.uint32).view(np.float32)[0]
            bot = np.array([(sw >> 16) << 16], np.uint32).view(np.float32)[0]
            assert top == S_orig[r0, c0 + j] and bot == S_orig[r0 + 4, c0 + j], (idx, j)
    lv = m._levels
    ts0 = pack_tiles(lv.shape, lv.sizes, lv.leaf, lv.modes, lv.scales, lv.codes_of, lv.scale_format, lv.row_perm,
                     lv.col_perm, gather_cols=False)
    assert not ts0.cols_gathered and ts0.col_perm is not None
    assert np.array_equal(_bits(decode_tiles(ts0)), _bits(_want(a, W)))
    with pytest.raises(ValueError):
        pack_tiles(lv.shape, lv.sizes, lv.leaf, lv.modes, lv.scales, lv.codes_of, lv.scale_format, lv.row_perm,
                   None, gather_cols=True)
