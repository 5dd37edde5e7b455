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
