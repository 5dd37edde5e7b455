"""On-disk form of a quadtree matrix (MTCMatrix.save / MTCMatrix.load).

A saved matrix keeps the allocation's grids, the permutations, the accounted bits and the
leaf codes; the weights and the allocator are not needed to load it. Bars: the loaded
matrix packs byte-identical panel and tile streams (so every GPU result is identical too),
its host-decoded W_hat equals the oracle's dequant of the original allocation bit for bit,
and the accounted size is unchanged. The reference keeps allocations in memory only, so
nothing of the reference pins the file layout itself: it is pinned by round trips.
"""

import numpy as np
import pytest

from oracle import mtc_oracle as O
from tensorpack_amd.core.permutation import PermutedQuadtreeRD
from tensorpack_amd.core.quadtree import QuadtreeRD
from tensorpack_amd.kernels.gemm import MTCMatrix
from tensorpack_amd.packer import PanelStream, decode_stream
from tensorpack_amd.tilestream import TileStream, decode_tiles

from conftest import outlier_matrix


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _same(a, b, cls):
    for f in cls.__dataclass_fields__:
        x, y = getattr(a, f), getattr(b, f)
        if isinstance(x, np.ndarray) or isinstance(y, np.ndarray):
            assert x is not None and y is not None and x.dtype == y.dtype and np.array_equal(x, y), f
        elif f != "stats":
            assert x == y, f


def _oracle_what(alloc, W):
    if hasattr(alloc, "inner"):
        i = alloc.inner
        return O.permuted_qt_dequant(W, alloc.row_perm, alloc.col_perm, i.sizes, i.leaf, i.modes, i.scales)
    return O.qt_dequant(W, alloc.sizes, alloc.leaf, alloc.modes, alloc.scales)


@pytest.mark.parametrize("permuted,budget", [(True, 3.125), (False, 4.25), (True, 11.0)])
def test_save_load_round_trip(tmp_path, permuted, budget):
    K, N = 192, 160
    W = outlier_matrix(7, K, N)
    h = np.exp(np.random.RandomState(8).randn(K))
    alloc = (PermutedQuadtreeRD if permuted else QuadtreeRD)(W, h, (32, 16, 8, 4)).select(budget)
    m = MTCMatrix.from_quadtree(alloc, W)
    path = tmp_path / "w.npz"
    m.save(path)
    back = MTCMatrix.load(path)
    assert back.shape == m.shape and back.total_bits == m.total_bits and back.is_quadtree
    for cr in (K, 64):
        _same(m.panel_stream(cr), back.panel_stream(cr), PanelStream)
    _same(m.tile_stream(), back.tile_stream(), TileStream)
    what = _oracle_what(alloc, W)
    assert np.array_equal(_bits(decode_stream(back.panel_stream(K))), _bits(what))
    # the tile stream holds bf16 weights for the MFMA path
    assert np.array_equal(_bits(decode_tiles(back.tile_stream())), _bits(O.bf16_round(what) + np.float32(0.0)))
    if budget > 8:                                    # some P16 leaves: the code grid is int16
        import zipfile
        with np.load(path, allow_pickle=False) as z:
            assert z["codes"].dtype == np.int16
        assert zipfile.is_zipfile(path)


def test_save_refuses_uniform_and_load_checks_format(tmp_path):
    from tensorpack_amd.core.allocation import rd_allocate
    W = outlier_matrix(3, 64, 64)
    a = rd_allocate(W, 4.0, block_size=16)
    u = MTCMatrix.from_allocation(W, a.modes, a.scales, 16)
    with pytest.raises(ValueError):
        u.save(tmp_path / "u.npz")
    alloc = QuadtreeRD(W, None, (32, 16, 8, 4)).select(4.0)
    m = MTCMatrix.from_quadtree(alloc, W)
    m.save(tmp_path / "m.npz")
    with np.load(tmp_path / "m.npz", allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files}
    arrays["format"] = np.array([99])
    np.savez(tmp_path / "bad.npz", **arrays)
    with pytest.raises(ValueError):
        MTCMatrix.load(tmp_path / "bad.npz")
    arrays["format"] = np.array([1])
    arrays["codes"] = arrays["codes"][:32]
    np.savez(tmp_path / "short.npz", **arrays)
    with pytest.raises(ValueError):
        MTCMatrix.load(tmp_path / "short.npz")


@pytest.mark.gpu
def test_loaded_matrix_on_gpu(gpu, tmp_path):
    from tensorpack_amd.kernels.gemm import mtc_gemm
    print("loaded matrix on gpu", flush=True)
    W = outlier_matrix(11, 256, 128)
    m = MTCMatrix.from_quadtree(PermutedQuadtreeRD(W, None, (32, 16, 8, 4)).select(4.0), W)
    m.save(tmp_path / "w.npz")
    back = MTCMatrix.load(tmp_path / "w.npz")
    for M in (1, 40):
        X = np.random.RandomState(M).randn(M, 256).astype(np.float32)
        assert np.array_equal(mtc_gemm(X, back), mtc_gemm(X, m)), M
    assert np.array_equal(back.to_array(), m.to_array())
