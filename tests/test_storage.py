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


def _resave(src, dst, **changes):
    """Copy an .npz, replacing the named arrays."""
    with np.load(src, allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files}
    arrays.update(changes)
    np.savez(dst, **arrays)


@pytest.fixture(scope="module")
def saved_qtp(tmp_path_factory):
    K, N = 128, 96
    W = outlier_matrix(11, K, N)
    h = np.exp(np.random.RandomState(12).randn(K))
    alloc = PermutedQuadtreeRD(W, h, (32, 16, 8, 4)).select(3.5)
    m = MTCMatrix.from_quadtree(alloc, W)
    d = tmp_path_factory.mktemp("qtp")
    m.save(d / "w.npz")
    m.panel_stream(64).save(d / "s.npz")
    return d, m


def test_load_rejects_corrupt_matrix(saved_qtp, tmp_path):
    """Permutations and codes index device memory: a file whose permutations are not
    permutations, whose modes or codes leave their ranges, or whose leaf grids overlap is
    refused before anything reaches the GPU."""
    d, m = saved_qtp
    src = d / "w.npz"
    with np.load(src, allow_pickle=False) as z:
        pr, pc, codes, leaf8, modes8 = z["row_perm"], z["col_perm"], z["codes"], z["leaf_8"], z["modes_8"]
    bad = {
        "row_perm out of range": {"row_perm": np.where(pr == 0, 128, pr)},
        "row_perm duplicate": {"row_perm": np.where(pr == 0, pr[1] if pr[0] != 0 else pr[0], pr)},
        "col_perm negative": {"col_perm": np.where(pc == 5, -1, pc)},
        "col_perm float": {"col_perm": pc.astype(np.float64)},
        "mode 7": {"modes_8": np.where(leaf8, 7, modes8).astype(np.uint8)},
        "overlapping leaves": {"leaf_8": np.ones_like(leaf8)},
    }
    wide = codes.astype(np.int16)
    wide[0, 0] = 20000                                # outside every width's range but P16
    bad["code out of range"] = {"codes": wide}
    for name, change in bad.items():
        dst = tmp_path / (name.replace(" ", "_") + ".npz")
        _resave(src, dst, **change)
        with pytest.raises(ValueError):
            MTCMatrix.load(dst)
    ok = tmp_path / "ok.npz"
    _resave(src, ok)
    assert MTCMatrix.load(ok).shape == m.shape


def test_panel_stream_load_rejects_corrupt_stream(saved_qtp, tmp_path):
    d, m = saved_qtp
    src = d / "s.npz"
    ps = PanelStream.load(src)
    ps.validate()
    hdr = ps.unit_hdr.copy()
    hdr[0, 1] = ps.payload.size                       # unit payload past the array
    bk = ps.buckets.copy()
    bk[0, 0] += 4 * ps.payload.size                   # bucket payload outside its unit
    bk2 = ps.buckets.copy()
    bk2[0, 3] = 7 | (2 << 8)                          # no leaf size 128
    lw = ps.leaf_word.copy()
    lw[:] |= 1023                                     # leaf rows past the unit's rows
    st1 = ps.steps.copy()
    st1[0, 3] ^= 1 << 8                               # slots of one record disagree on the kind word
    st2 = ps.steps.copy()
    st2[0, 1::2] = (st2[0, 1::2] & ~np.uint32(0xF8)) | np.uint32(7 << 3)   # code width 7
    st3 = ps.steps.copy()
    st3[0, 1::2] |= np.uint32(17 << 8)                # 17+ chunks in a 16-chunk step
    h4 = ps.unit_hdr.copy()
    h4[0, 28] = 60000                                 # a block with more records than the array holds
    h4[0, 27] = 100000000
    h5 = ps.unit_hdr.copy()
    h5[0, 28] = ps.fixed_steps + 2                    # overflow records starting inside the fixed area
    h5[0, 27] = 0
    st4 = ps.steps.copy()
    st4[:, 0::2] = np.uint32(0xFFFFFFFF)              # every slot word at the end of the 16-bit ranges
    st5 = ps.steps.copy()
    on = np.nonzero(((st5[:, 1].astype(np.int64) >> 8) & 31) > 0)[0][0]
    st5[on, 0] = (st5[on, 0] & np.uint32(0xFFFF)) | np.uint32(0xFFF0 << 16)   # first leaf past the unit
    st6 = ps.steps.copy()
    st6[on, 0] = (st6[on, 0] & np.uint32(0xFFFF0000)) | np.uint32(0xFFF0)     # payload past the unit
    st7 = ps.steps.copy()
    st7[ps.unit_hdr.shape[0] * 2 * ps.fixed_steps, 1::2] |= np.uint32(1 << 8)  # a chunk in the null record
    bad = {"hdr": {"unit_hdr": hdr}, "bucket payload": {"buckets": bk}, "bucket kind": {"buckets": bk2},
           "leaf rows": {"leaf_word": lw}, "row_perm": {"row_perm": np.zeros_like(ps.row_perm)},
           "col_perm": {"col_perm": ps.col_perm + 1}, "record kind words": {"steps": st1},
           "record width": {"steps": st2}, "record count": {"steps": st3},
           "block record count": {"unit_hdr": h4}, "overflow start": {"unit_hdr": h5},
           "slot words": {"steps": st4}, "slot leaf": {"steps": st5}, "slot payload": {"steps": st6},
           "null record": {"steps": st7}}
    for name, change in bad.items():
        dst = tmp_path / (name.replace(" ", "_") + ".npz")
        _resave(src, dst, **change)
        with pytest.raises(ValueError):
            PanelStream.load(dst)
