"""GPU parity of the HIP path against the CPU oracle (run on an MI355X).

Bars: W_hat bit-exact vs the oracle's qt_dequant (-0.0 == +0.0
never arises: the quadtree W_hat has no negative zeros); Y within relative
Frobenius 1e-5 of fp64 X @ W_hat for the fp32 path and 2e-3 for the bf16
MFMA path (fp64 reference built from the same bf16-rounded X).
"""

import ctypes

import numpy as np
import pytest

from oracle import mtc_oracle as O
from tensorpack_amd.core.allocation import rd_allocate, rd_allocate_pair
from tensorpack_amd.core.permutation import PermutedQuadtreeRD
from tensorpack_amd.core.quadtree import QuadtreeRD
from tensorpack_amd.kernels.gemm import F32_DECODE_MAX_M, MTCMatrix, mtc_gemm

from conftest import kind_grid_stream, kind_mix_stream, largest_unit_stream, outlier_matrix, signed_scale_levels

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5
TOL_BF16 = 2e-3


def _say(*a):
    print(*a, flush=True)


def _oracle_what(alloc, W):
    """Oracle W_hat (original channel order) of a QT or QT-P allocation of W."""
    if hasattr(alloc, "inner"):
        i = alloc.inner
        return O.permuted_qt_dequant(W, alloc.row_perm, alloc.col_perm, i.sizes, i.leaf, i.modes, i.scales)
    return O.qt_dequant(W, alloc.sizes, alloc.leaf, alloc.modes, alloc.scales)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


CASES = [
    # name, K, N, seed, permuted, budget, sizes
    ("outlier-qt-2.5", 256, 256, 1, False, 2.5, (32, 16, 8, 4)),
    ("outlier-qtp-4.25", 256, 384, 2, True, 4.25, (32, 16, 8, 4)),
    ("outlier-qt-9", 192, 128, 3, False, 9.0, (32, 16, 8, 4)),
    ("qt-p16-heavy", 128, 96, 4, False, 14.0, (32, 16, 8, 4)),
    ("qtp-2.2-root16", 320, 160, 5, True, 2.2, (16, 8, 4)),
]


@pytest.fixture(scope="module")
def allocs():
    out = {}
    for name, K, N, seed, perm, budget, sizes in CASES:
        W = outlier_matrix(seed, K, N)
        h = np.exp(np.random.RandomState(seed + 100).randn(K))
        cls = PermutedQuadtreeRD if perm else QuadtreeRD
        a = cls(W, h, sizes).select(budget)
        out[name] = (W, a, MTCMatrix.from_quadtree(a, W))
    return out


@pytest.mark.parametrize("name", [c[0] for c in CASES])
def test_dequant_bit_exact(gpu, allocs, name):
    W, a, m = allocs[name]
    _say("dequant", name)
    got = m.to_array()
    ref = _oracle_what(a, W)
    assert np.array_equal(_bits(got), _bits(ref)), name
    assert not np.signbit(got[got == 0]).any()


@pytest.mark.parametrize("chunk_rows", [32, 64, 160, 512])
def test_dequant_any_chunking(gpu, allocs, chunk_rows):
    W, a, m = allocs["outlier-qtp-4.25"]
    _say("dequant chunking", chunk_rows)
    got = m.device_stream(chunk_rows).dequant().cpu().numpy()
    assert np.array_equal(_bits(got), _bits(_oracle_what(a, W)))


@pytest.mark.parametrize("name", [c[0] for c in CASES])
@pytest.mark.parametrize("M", [1, 2, 3, 5, 8, 12, 16, 17, 40])
def test_gemv_f32(gpu, allocs, name, M):
    import torch
    W, a, m = allocs[name]
    _say("gemv", name, M)
    X = np.random.RandomState(M).randn(M, W.shape[0]).astype(np.float32)
    Y = mtc_gemm(torch.from_numpy(X).to(gpu), m, compute="fp32").cpu().numpy()
    ref = O.qt_gemm_f64(X, _oracle_what(a, W))
    err = O.relative_frobenius_error(ref, Y)
    assert err <= TOL_F32, (name, M, err)


@pytest.mark.parametrize("name", [c[0] for c in CASES])
@pytest.mark.parametrize("M", [1, 2, 5, 16])
def test_gemv_f32_mx_layout(gpu, allocs, name, M):
    """The matrix-core payload layout (opt-in, one X row per block): W_hat bit-exact and Y
    within the fp32 bar, at the decode layout's row chunks and at split-K chunkings."""
    import torch
    from tensorpack_amd.packer import LAYOUT_MX
    W, a, m = allocs[name]
    X = np.random.RandomState(50 + M).randn(M, W.shape[0]).astype(np.float32)
    Xd = torch.from_numpy(X).to(gpu)
    ref = O.qt_gemm_f64(X, _oracle_what(a, W))
    for cr in (None, 64):
        _say("gemv mx", name, M, cr)
        ds = m.device_stream(cr, gpu, 1, LAYOUT_MX)
        if M == 1:
            got = ds.dequant().cpu().numpy()
            assert np.array_equal(_bits(got), _bits(_oracle_what(a, W))), (name, cr)
        Y = ds.gemv_f32(Xd).cpu().numpy()
        err = O.relative_frobenius_error(ref, Y)
        assert err <= TOL_F32, (name, M, cr, err)


@pytest.mark.parametrize("chunk_rows", [32, 64, 96, 512])
@pytest.mark.parametrize("M", [4, 12])
def test_gemv_split_k_chunkings(gpu, allocs, chunk_rows, M):
    import torch
    W, a, m = allocs["outlier-qt-2.5"]
    _say("gemv chunking", chunk_rows, M)
    X = np.random.RandomState(7).randn(M, W.shape[0]).astype(np.float32)
    ds = m.device_stream(chunk_rows)
    Y1 = ds.gemv_f32(torch.from_numpy(X).to(gpu)).cpu().numpy()
    Y2 = ds.gemv_f32(torch.from_numpy(X).to(gpu)).cpu().numpy()
    assert np.array_equal(Y1, Y2), "fp32 path must be deterministic (counters must self-reset)"
    err = O.relative_frobenius_error(O.qt_gemm_f64(X, _oracle_what(a, W)), Y1)
    assert err <= TOL_F32, err


@pytest.mark.parametrize("name", [c[0] for c in CASES])
def test_gemv_matrix_core_tile_heights_agree(gpu, allocs, name):
    # M tiles of 8 and 16 rows run the same lane -> chunk order: the rows both compute are
    # bit-identical, and every M from 5 to 16 matches the 16-row call's rows
    import torch
    W, a, m = allocs[name]
    ds = m.device_stream(512, gpu)
    X = torch.from_numpy(np.random.RandomState(11).randn(16, W.shape[0]).astype(np.float32)).to(gpu)
    _say("gemv tile heights", name)
    Y16 = ds.gemv_f32(X).cpu().numpy()
    for M in (5, 8, 9, 13):
        Y = ds.gemv_f32(X[:M].contiguous()).cpu().numpy()
        assert np.array_equal(_bits(Y), _bits(Y16[:M])), (name, M)


def test_gemm_short_row_tiles(gpu):
    """Single prefill calls with M <= 256 and few output tiles run blocks of fewer output rows
    (the tile plan prices 64- and 128-row blocks against 256-row ones; at this shape it takes
    64 rows, and the c5 configuration test at M = 256 runs 128-row blocks): Y is within the
    bf16 bar at every M around the tile heights, and a group call, which runs the same K split
    with 256-row tiles, gives the same Y bit for bit."""
    import torch
    from tensorpack_amd.device import gemm_bf16_group
    K, N = 2048, 512
    W = outlier_matrix(41, K, N)
    a = PermutedQuadtreeRD(W, np.exp(np.random.RandomState(42).randn(K)), (32, 16, 8, 4)).select(3.5)
    m = MTCMatrix.from_quadtree(a, W)
    g = m.device_tiles(gpu)
    ref_w = _oracle_what(a, W)
    for M in (1, 40, 64, 65, 100, 128, 129, 200, 256):
        _say("gemm short row tiles", M)
        X = np.random.RandomState(M + 3).randn(M, K).astype(np.float32)
        Xb = torch.from_numpy(X).to(gpu).to(torch.bfloat16)
        Y = g.gemm_bf16(Xb).cpu().numpy()
        err = O.relative_frobenius_error(O.qt_gemm_f64(Xb.float().cpu().numpy(), ref_w), Y)
        assert err <= TOL_BF16, (M, err)
        Yg = gemm_bf16_group([g], Xb)[0].cpu().numpy()
        assert np.array_equal(_bits(Yg), _bits(Y)), M


@pytest.mark.parametrize("K,ldx", [(2048, 2048), (992, 992), (992, 995)])
def test_gemm_fp32_x_read_in_place(gpu, K, ldx):
    """fp32 X without a row permutation, at M <= 256 (tiles of 64 or 128 rows): the tile
    kernel's consumers round X to bf16 themselves instead of a staging launch. Y equals the
    call on bf16(X) bit for bit (one split and split K, a partial last K-step at K = 992), and
    rows not 16-byte aligned (ldx = 995) take the staging launch with the same Y."""
    import torch
    N = 512
    W = outlier_matrix(61, K, N)
    a = QuadtreeRD(W, None, (32, 16, 8, 4)).select(3.5)
    m = MTCMatrix.from_quadtree(a, W)
    g = m.device_tiles(gpu)
    ref_w = _oracle_what(a, W)
    for M in (1, 37, 64, 100, 128, 200, 256):
        _say("gemm fp32 X in place", K, ldx, M)
        X = np.random.RandomState(M + 5).randn(M, K).astype(np.float32)
        big = torch.zeros(M, ldx, device=gpu)
        big[:, :K] = torch.from_numpy(X).to(gpu)
        Xf = big[:, :K]
        Yf = g.gemm_bf16(Xf).cpu().numpy()
        Yb = g.gemm_bf16(Xf.to(torch.bfloat16).contiguous()).cpu().numpy()
        assert np.array_equal(_bits(Yf), _bits(Yb)), (K, ldx, M)
        err = O.relative_frobenius_error(O.qt_gemm_f64(O.bf16_round(X), ref_w), Yf)
        assert err <= TOL_BF16, (K, ldx, M, err)


@pytest.mark.parametrize("M,permuted,ydt", [(100, False, "f32"), (300, True, "f32"), (37, True, "bf16")])
def test_gemm_split_k(gpu, M, permuted, ydt):
    # few output tiles and 32 K-steps: the K steps are split over blocks and the fp32
    # partial tiles summed (and column-permuted) by the reduce kernel
    import torch
    K, N = 2048, 256
    W = outlier_matrix(31, K, N)
    cls = PermutedQuadtreeRD if permuted else QuadtreeRD
    a = cls(W, np.exp(np.random.RandomState(32).randn(K)), (32, 16, 8, 4)).select(4.5)
    m = MTCMatrix.from_quadtree(a, W)
    g = m.device_tiles(gpu)
    need = g.lib.mtc_gemm_workspace_bytes(ctypes.byref(g.desc), M, 1)
    assert need >= 4 * M * N * 2, need                     # at least two fp32 partial tiles
    _say("gemm split-K", M, permuted, ydt)
    X = np.random.RandomState(M).randn(M, K).astype(np.float32)
    Xb = torch.from_numpy(X).to(gpu).to(torch.bfloat16)
    out_dtype = torch.float32 if ydt == "f32" else torch.bfloat16
    Y1 = g.gemm_bf16(Xb, out_dtype=out_dtype).float().cpu().numpy()
    Y2 = g.gemm_bf16(Xb, out_dtype=out_dtype).float().cpu().numpy()
    assert np.array_equal(Y1, Y2), "split-K reduction must be deterministic"
    ref = O.qt_gemm_f64(Xb.float().cpu().numpy(), _oracle_what(a, W))
    err = O.relative_frobenius_error(ref, Y1)
    assert err <= TOL_BF16, err


@pytest.mark.parametrize("M", [1, 2, 4, 7])
def test_gemv_step_records_past_the_fixed_area(gpu, M):
    # blocks with more step records than the fixed area (overflow list read via the header)
    import torch
    from tensorpack_amd.device import DeviceStream
    from tensorpack_amd.packer import MAX_FIXED_STEPS, decode_stream
    ps = kind_mix_stream()
    assert max(ps.unit_hdr[:, 28].max(), ps.unit_hdr[:, 30].max()) > MAX_FIXED_STEPS
    _say("gemv overflow records", M)
    X = np.random.RandomState(M + 40).randn(M, ps.K).astype(np.float32)
    Y = DeviceStream(ps, gpu).gemv_f32(torch.from_numpy(X).to(gpu)).cpu().numpy()
    err = O.relative_frobenius_error(O.qt_gemm_f64(X, decode_stream(ps)), Y)
    assert err <= TOL_F32, err


def test_largest_unit(gpu):
    """One 4096-row unit of P16 4x4 leaves (65536 payload dwords, 8192 leaf words: the step
    records' unit-relative offsets at their largest): dequant bit-exact, Y within the fp32 bar
    for M = 1, 2, 4 (vector path) and 8 (matrix core)."""
    import torch
    from tensorpack_amd.device import DeviceStream
    ps, W_hat = largest_unit_stream()
    ds = DeviceStream(ps, gpu)
    _say("largest unit")
    got = ds.dequant().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), W_hat.view(np.uint32))
    for M in (1, 2, 4, 8):
        X = np.random.RandomState(M + 90).randn(M, ps.K).astype(np.float32)
        Y = ds.gemv_f32(torch.from_numpy(X).to(gpu)).cpu().numpy()
        err = O.relative_frobenius_error(O.qt_gemm_f64(X, W_hat), Y)
        assert err <= TOL_F32, (M, err)


@pytest.mark.parametrize("S", [8, 16, 32])
@pytest.mark.parametrize("merge", [False, True])
def test_every_kind_of_a_leaf_size(gpu, S, merge):
    """Every code width at leaf size S in every unit (kind_grid_stream), stored at its own
    width or merged into wider ones: the dequant is bit-exact against the host decode of the
    same stream, and Y is within the fp32 bar on the vector path (M = 1, 2) and on the matrix
    core (M = 5, 16)."""
    import torch
    from tensorpack_amd.device import DeviceStream
    from tensorpack_amd.packer import decode_stream
    ps = kind_grid_stream(S, merge_kinds=merge)
    kinds = {(int(k) & 0xFF, int(k) >> 8) for k in ps.buckets[:ps.n_buckets, 3]}
    assert merge or len(kinds) == 7, kinds                 # every width present unmerged
    ref = decode_stream(ps)
    ds = DeviceStream(ps, gpu)
    _say("every kind", S, merge)
    got = ds.dequant().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    for M in (1, 2, 5, 16):
        X = np.random.RandomState(M + S).randn(M, ps.K).astype(np.float32)
        Y = ds.gemv_f32(torch.from_numpy(X).to(gpu)).cpu().numpy()
        err = O.relative_frobenius_error(O.qt_gemm_f64(X, ref), Y)
        assert err <= TOL_F32, (S, merge, M, err)


def test_all_p0_matrix_and_empty_x(gpu, allocs):
    """A matrix whose every leaf is P0 stores no codes (no buckets, only the null record): the
    dequant is all +0.0 and Y is all zero on the vector path, the matrix core and the prefill.
    An X of M = 0 rows gives a (0, N) Y on the decode and the prefill paths."""
    import torch
    from tensorpack_amd.device import DeviceStream, DeviceTiles
    from tensorpack_amd.packer import pack_levels
    from tensorpack_amd.tilestream import pack_tiles
    _say("all P0 / empty X")
    K, N = 256, 96
    grids = ((K, N), (16, 4), {16: np.ones((K // 16, N // 16), bool), 4: np.zeros((K // 4, N // 4), bool)},
             {16: np.zeros((K // 16, N // 16), np.int64), 4: np.zeros((K // 4, N // 4), np.int64)},
             {16: np.ones((K // 16, N // 16), np.float32), 4: np.ones((K // 4, N // 4), np.float32)},
             lambda *a: None)
    ps = pack_levels(*grids, chunk_rows=128)
    assert ps.n_buckets == 0
    ds = DeviceStream(ps, gpu)
    w = ds.dequant().cpu().numpy()
    assert np.array_equal(w.view(np.uint32), np.zeros((K, N), np.uint32))
    for M in (1, 3, 9):
        X = torch.from_numpy(np.random.RandomState(M).randn(M, K).astype(np.float32)).to(gpu)
        Y = ds.gemv_f32(X).cpu().numpy()
        assert Y.shape == (M, N) and not Y.any(), M
    Yb = DeviceTiles(pack_tiles(*grids), gpu).gemm_bf16(torch.ones((40, K), device=gpu, dtype=torch.bfloat16))
    assert Yb.shape == (40, N) and not Yb.float().cpu().numpy().any()
    W, a, m = allocs[CASES[0][0]]
    for compute in ("fp32", "bf16"):
        Y0 = mtc_gemm(torch.zeros((0, W.shape[0]), device=gpu), m, compute=compute)
        assert tuple(Y0.shape) == (0, W.shape[1]), compute


def test_negative_scales(gpu):
    """Scales may be negative (any sign of s gives W_hat = q * s): the dequant is bit-exact
    against W_hat built from the leaf grids directly, the decode is within the fp32 bar on
    the vector path and the matrix core, and the prefill within the bf16 bar."""
    import torch
    from tensorpack_amd.device import DeviceStream, DeviceTiles
    from tensorpack_amd.packer import pack_levels
    from tensorpack_amd.tilestream import pack_tiles
    args, W_hat = signed_scale_levels()
    _say("negative scales")
    ds = DeviceStream(pack_levels(*args, chunk_rows=256), gpu)
    got = ds.dequant().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), W_hat.view(np.uint32))
    for M in (1, 2, 5, 16):
        X = np.random.RandomState(M + 70).randn(M, W_hat.shape[0]).astype(np.float32)
        Y = ds.gemv_f32(torch.from_numpy(X).to(gpu)).cpu().numpy()
        err = O.relative_frobenius_error(O.qt_gemm_f64(X, W_hat), Y)
        assert err <= TOL_F32, (M, err)
    dt = DeviceTiles(pack_tiles(*args), gpu)
    for M in (1, 64, 300):
        X = np.random.RandomState(M + 80).randn(M, W_hat.shape[0]).astype(np.float32)
        Y = dt.gemm_bf16(torch.from_numpy(X).to(gpu).to(torch.bfloat16)).float().cpu().numpy()
        err = O.relative_frobenius_error(O.qt_gemm_f64(O.bf16_round(X), W_hat), Y)
        assert err <= TOL_BF16, (M, err)


@pytest.mark.parametrize("name", [c[0] for c in CASES])
@pytest.mark.parametrize("M", [1, 31, 128, 200])
@pytest.mark.parametrize("xdtype", ["f32", "bf16"])
def test_gemm_bf16(gpu, allocs, name, M, xdtype):
    import torch
    W, a, m = allocs[name]
    _say("gemm", name, M, xdtype)
    X = np.random.RandomState(M + 1).randn(M, W.shape[0]).astype(np.float32)
    Xt = torch.from_numpy(X).to(gpu)
    if xdtype == "bf16":
        Xt = Xt.to(torch.bfloat16)
    Y = mtc_gemm(Xt, m, compute="bf16").float().cpu().numpy()
    ref = O.qt_gemm_f64(O.bf16_round(X), _oracle_what(a, W))
    err = O.relative_frobenius_error(ref, Y)
    assert err <= TOL_BF16, (name, M, err)


@pytest.mark.parametrize("name", [c[0] for c in CASES])
@pytest.mark.parametrize("M", [1, 5, 16, 17, 40])
def test_gemm_f32_tiles(gpu, allocs, name, M):
    """The fp32 matrix-core path over the tile stream (mtc_gemm_f32: exact W_hat, fp32 products
    and sums, 16-row tiles, split K): Y within the fp32 bar, every call the same bits, and X = I
    returns W_hat itself (one product per output, exact in fp32)."""
    import torch
    W, a, m = allocs[name]
    t = m.device_tiles(gpu)
    _say("gemm f32 tiles", name, M)
    X = np.random.RandomState(M + 90).randn(M, W.shape[0]).astype(np.float32)
    Xd = torch.from_numpy(X).to(gpu)
    Y = t.gemm_f32(Xd).cpu().numpy()
    ref = O.qt_gemm_f64(X, _oracle_what(a, W))
    err = O.relative_frobenius_error(ref, Y)
    assert err <= TOL_F32, (name, M, err)
    assert np.array_equal(_bits(t.gemm_f32(Xd).cpu().numpy()), _bits(Y)), (name, M)
    if M > F32_DECODE_MAX_M:                     # mtc_gemm's fp32 path above 16 rows is this kernel
        assert np.array_equal(_bits(mtc_gemm(Xd, m, compute="fp32").cpu().numpy()), _bits(Y)), (name, M)
        # a view whose rows are not 16-byte aligned is copied first, with the same result
        big = torch.zeros((M, W.shape[0] + 1), device=gpu)
        big[:, 1:] = Xd
        assert np.array_equal(_bits(mtc_gemm(big[:, 1:], m, compute="fp32").cpu().numpy()), _bits(Y)), (name, M)
    if M == 1:
        K = W.shape[0]
        Yi = t.gemm_f32(torch.eye(K, device=gpu)).cpu().numpy()
        want = _oracle_what(a, W) + np.float32(0.0)
        assert np.array_equal(_bits(Yi), _bits(want)), name


@pytest.mark.parametrize("name", [c[0] for c in CASES])
def test_gemm_stages_bf16_w_hat_exactly(gpu, allocs, name):
    """X = I makes the MFMA path return its staged weight tile: it must equal
    bf16(W_hat) bit for bit (a single product per output, exact in fp32)."""
    import torch
    W, a, m = allocs[name]
    _say("gemm identity", name)
    K = W.shape[0]
    I = torch.eye(K, device=gpu, dtype=torch.bfloat16)
    Y = mtc_gemm(I, m, compute="bf16").cpu().numpy()
    want = O.bf16_round(_oracle_what(a, W)) + np.float32(0.0)
    assert np.array_equal(_bits(Y), _bits(want)), name
    # fp32 X (staged to bf16 on the device) gives the same
    Y32 = mtc_gemm(I.float(), m, compute="bf16").cpu().numpy()
    assert np.array_equal(_bits(Y32), _bits(want)), name


@pytest.mark.parametrize("M", [255, 257, 600])
def test_gemm_bf16_row_tiles(gpu, allocs, M):
    import torch
    W, a, m = allocs["outlier-qtp-4.25"]
    _say("gemm row tiles", M)
    X = np.random.RandomState(M).randn(M, W.shape[0]).astype(np.float32)
    Y = mtc_gemm(torch.from_numpy(X).to(gpu).to(torch.bfloat16), m, compute="bf16").cpu().numpy()
    err = O.relative_frobenius_error(O.qt_gemm_f64(O.bf16_round(X), _oracle_what(a, W)), Y)
    assert err <= TOL_BF16, (M, err)


def test_gemm_partial_k_step_and_strided_x(gpu):
    """K = 96 (a 64-row step and a half step), N = 64, X a strided view."""
    import torch
    W = outlier_matrix(21, 96, 64)
    a = QuadtreeRD(W, None, (32, 16, 8, 4)).select(5.0)
    m = MTCMatrix.from_quadtree(a, W)
    big = torch.randn(70, 104, device=gpu, dtype=torch.bfloat16)
    X = big[:, :96]                                               # ldx = 104
    Y = mtc_gemm(X, m, compute="bf16").cpu().numpy()
    ref = O.qt_gemm_f64(X.float().cpu().numpy(), _oracle_what(a, W))
    assert O.relative_frobenius_error(ref, Y) <= TOL_BF16


def test_gemm_uniform_form_fp32_scales(gpu):
    import torch
    rng = np.random.RandomState(8)
    W = rng.randn(256, 128).astype(np.float32)
    al = rd_allocate(W, 4.0, None, 32)
    m = MTCMatrix.from_allocation(W, al.modes, al.scales, 32)
    W_hat = O.uniform_to_array(W, al.modes, al.scales, 32)
    X = rng.randn(300, 256).astype(np.float32)
    Y = mtc_gemm(torch.from_numpy(X).to(gpu), m, compute="bf16").cpu().numpy()
    assert O.relative_frobenius_error(O.qt_gemm_f64(O.bf16_round(X), W_hat), Y) <= TOL_BF16
    I = torch.eye(256, device=gpu, dtype=torch.bfloat16)
    Yi = mtc_gemm(I, m, compute="bf16").cpu().numpy()
    assert np.array_equal(_bits(Yi), _bits(O.bf16_round(W_hat) + np.float32(0.0)))


def test_gemm_bf16_output(gpu, allocs):
    import torch
    W, a, m = allocs["outlier-qt-2.5"]
    X = torch.randn(64, W.shape[0], device=gpu, dtype=torch.bfloat16)
    Y = mtc_gemm(X, m, compute="bf16", out_dtype=torch.bfloat16)
    assert Y.dtype == torch.bfloat16 and Y.shape == (64, W.shape[1])
    ref = O.qt_gemm_f64(X.float().cpu().numpy(), _oracle_what(a, W))
    assert O.relative_frobenius_error(ref, Y.float().cpu().numpy()) <= TOL_BF16 + 4e-3


def test_numpy_in_numpy_out_and_vector(gpu, allocs):
    W, a, m = allocs["outlier-qtp-4.25"]
    x = np.random.RandomState(3).randn(W.shape[0]).astype(np.float32)
    y = mtc_gemm(x, m)
    assert isinstance(y, np.ndarray) and y.shape == (W.shape[1],)
    ref = O.qt_gemm_f64(x[None], _oracle_what(a, W))[0]
    assert O.relative_frobenius_error(ref, y) <= TOL_F32


def test_all_p0_and_single_mode_edges(gpu):
    """All-P0 (budget floor), every element one 4x4 P16 leaf, negative scales."""
    W = outlier_matrix(9, 64, 64)
    W[:, :32] = 0.0                       # an all-zero panel -> P0 leaves everywhere in it
    a = QuadtreeRD(W, None, (32, 16, 8, 4)).select(1.0)
    m = MTCMatrix.from_quadtree(a, W)
    ref = O.qt_dequant(W, a.sizes, a.leaf, a.modes, a.scales)
    assert np.array_equal(_bits(m.to_array()), _bits(ref))
    X = np.random.RandomState(1).randn(2, 64).astype(np.float32)
    assert O.relative_frobenius_error(O.qt_gemm_f64(X, ref), mtc_gemm(X, m)) <= TOL_F32
    # a budget high enough for P16 everywhere
    b = QuadtreeRD(W, None, (4,)).select(17.5)
    assert all((b.modes[4][b.leaf[4]] == 16) | (b.modes[4][b.leaf[4]] == 0))
    mb = MTCMatrix.from_quadtree(b, W)
    refb = O.qt_dequant(W, b.sizes, b.leaf, b.modes, b.scales)
    assert np.array_equal(_bits(mb.to_array()), _bits(refb))
    assert O.relative_frobenius_error(O.qt_gemm_f64(X, refb), mtc_gemm(X, mb)) <= TOL_F32


def test_uniform_form_packed_kernel_matches_simulation(gpu):
    """tests/test_allocation.py:69-86 on the GPU: arena round trip exact, GEMM < 1e-5."""
    for budget in (2.6, 3.3, 5.2, 6.3, 9.0):
        rng = np.random.RandomState(5)
        A = rng.randn(128, 96).astype(np.float32)
        B = rng.randn(96, 64).astype(np.float32)
        A[:, :32] *= 1e-4
        B[32:64] *= 20.0
        a, b = rd_allocate_pair(A, B, budget)
        Am = MTCMatrix.from_allocation(A, a.modes, a.scales, 16)
        Bm = MTCMatrix.from_allocation(B, b.modes, b.scales, 16)
        A_hat = O.uniform_to_array(A, a.modes, a.scales, 16)
        B_hat = O.uniform_to_array(B, b.modes, b.scales, 16)
        assert np.array_equal(_bits(Am.to_array()), _bits(A_hat))
        assert np.array_equal(_bits(Bm.to_array()), _bits(B_hat))
        # the allocator's W_hat as values (it keeps np.round's -0.0 where the arena holds code 0)
        assert np.array_equal(Am.to_array(), O.uniform_dequant(A, a.modes, a.scales, 16))
        C_sim = A_hat.astype(np.float64) @ B_hat.astype(np.float64)
        assert O.relative_frobenius_error(C_sim, mtc_gemm(Am, Bm)) < 1e-5
        assert Am.total_bytes_allocated * 8 == a.payload_bits
        assert Bm.total_bytes_allocated * 8 == b.payload_bits


@pytest.mark.parametrize("M", [3, 9, 16])          # vector decode; matrix core at 9 and 16
def test_uniform_form_dense_x(gpu, M):
    rng = np.random.RandomState(8)
    W = rng.randn(256, 128).astype(np.float32)
    al = rd_allocate(W, 4.0, None, 32)
    m = MTCMatrix.from_allocation(W, al.modes, al.scales, 32)
    X = rng.randn(M, 256).astype(np.float32)
    W_hat = O.uniform_to_array(W, al.modes, al.scales, 32)
    assert O.relative_frobenius_error(O.qt_gemm_f64(X, W_hat), mtc_gemm(X, m)) <= TOL_F32


@pytest.mark.parametrize("M", [1, 3])
def test_uniform_form_mx_layout(gpu, M):
    """The uniform-block form (fp32 scales) in the matrix-core payload layout: dequant bit for bit
    against the reference's to_array, Y within the fp32 bar."""
    import torch
    from tensorpack_amd.packer import LAYOUT_MX
    rng = np.random.RandomState(18)
    W = rng.randn(256, 128).astype(np.float32)
    al = rd_allocate(W, 5.0, None, 16)
    m = MTCMatrix.from_allocation(W, al.modes, al.scales, 16)
    W_hat = O.uniform_to_array(W, al.modes, al.scales, 16)
    ds = m.device_stream(None, gpu, 1, LAYOUT_MX)
    assert ds.host.leaf_scale is not None                   # the fp32-scale kernels
    assert np.array_equal(_bits(ds.dequant().cpu().numpy()), _bits(W_hat))
    X = rng.randn(M, 256).astype(np.float32)
    Y = ds.gemv_f32(torch.from_numpy(X).to(gpu)).cpu().numpy()
    assert O.relative_frobenius_error(O.qt_gemm_f64(X, W_hat), Y) <= TOL_F32


def test_errors_are_clean(gpu, allocs):
    import ctypes
    import torch
    from tensorpack_amd import _abi
    W, a, m = allocs["outlier-qt-2.5"]
    with pytest.raises(ValueError):
        mtc_gemm(torch.zeros(2, W.shape[0] + 1, device=gpu), m)
    ds = m.device_stream(None)
    lib = ds.lib
    X = torch.zeros(1, W.shape[0], device=gpu)
    Y = torch.zeros(1, W.shape[1], device=gpu)
    assert lib.mtc_gemv_f32(ctypes.byref(ds.desc), None, W.shape[0], Y.data_ptr(), W.shape[1], 1, None, 0, None) == -1
    assert lib.mtc_gemv_f32(ctypes.byref(ds.desc), X.data_ptr(), W.shape[0], Y.data_ptr(), W.shape[1], 0, None, 0,
                            None) == -3
    bad = _abi.MtcStreamDesc()
    assert lib.mtc_gemv_f32(ctypes.byref(bad), X.data_ptr(), W.shape[0], Y.data_ptr(), W.shape[1], 1, None, 0,
                            None) == -7
    assert b"ABI" in lib.mtc_last_error()
    g = m.device_tiles()
    assert lib.mtc_gemm_bf16(ctypes.byref(g.desc), X.data_ptr(), 7, W.shape[0], Y.data_ptr(), 0, W.shape[1], 1,
                             None, 0, None) == -4
    # fp32 X needs the bf16 staging workspace
    assert lib.mtc_gemm_bf16(ctypes.byref(g.desc), X.data_ptr(), 0, W.shape[0], Y.data_ptr(), 0, W.shape[1], 1,
                             None, 0, None) == -5
    Xb = torch.zeros(1, W.shape[0] + 1, device=gpu, dtype=torch.bfloat16)
    assert lib.mtc_gemm_bf16(ctypes.byref(g.desc), Xb.data_ptr(), 1, W.shape[0] + 1, Y.data_ptr(), 0, W.shape[1],
                             1, None, 0, None) == -3                                  # rows not 16-byte aligned
