"""Prefill on the decode-once path (run on an MI355X): calls with at least max(512, K / 8) rows
of X and no output column permutation decode W_hat once into bf16 (k_tile_dequant_bf16) and
multiply it with hipBLASLt's bf16 GEMM (fp32 accumulation).

Bars: the decoded bf16 W_hat bit-exact against bf16(oracle W_hat) in the stream's row order;
Y within 2e-3 relative Frobenius of the fp64 product of the same bf16 X (the bf16 path's
bar) and within 1e-5 of the fused tile kernel's Y (the same bf16 operands, fp32 sums in
another order); repeated calls and group members bit-identical to single calls.
"""

import ctypes

import numpy as np
import pytest

from oracle import mtc_oracle as O
from tensorpack_amd import _abi
from tensorpack_amd.core.allocation import rd_allocate
from tensorpack_amd.core.permutation import PermutedQuadtreeRD
from tensorpack_amd.core.quadtree import QuadtreeRD
from tensorpack_amd.kernels.gemm import MTCMatrix

from conftest import outlier_matrix

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-3
K, N, M = 1024, 4096, 4096          # eligible from 512 rows on


def _say(*a):
    print(*a, flush=True)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def mats():
    """QT (bf16 scale pairs), QT-P (gathered columns, row permutation) and the uniform form
    (fp32 scales): one of each cell format, with the oracle's W_hat in the original order."""
    W = outlier_matrix(71, K, N)
    h = np.exp(np.random.RandomState(72).randn(K))
    out = {}
    a = QuadtreeRD(W, h, (32, 16, 8, 4)).select(4.5)
    out["qt"] = (MTCMatrix.from_quadtree(a, W), O.qt_dequant(W, a.sizes, a.leaf, a.modes, a.scales))
    p = PermutedQuadtreeRD(W, h, (32, 16, 8, 4)).select(3.5)
    i = p.inner
    out["qtp"] = (MTCMatrix.from_quadtree(p, W),
                  O.permuted_qt_dequant(W, p.row_perm, p.col_perm, i.sizes, i.leaf, i.modes, i.scales))
    al = rd_allocate(W, 4.0, None, 32)
    out["uniform"] = (MTCMatrix.from_allocation(W, al.modes, al.scales, 32), O.uniform_to_array(W, al.modes, al.scales, 32))
    return out


@pytest.fixture(scope="module")
def xs(gpu):
    import torch
    X = np.random.RandomState(73).randn(M, K).astype(np.float32)
    Xf = torch.from_numpy(X).to(gpu)
    return Xf, Xf.to(torch.bfloat16)


def _fused(fn):
    from tensorpack_amd.device import set_prefill_decode_once
    prev = set_prefill_decode_once(False)
    try:
        return fn()
    finally:
        set_prefill_decode_once(prev)


@pytest.mark.parametrize("name", ["qt", "qtp", "uniform"])
def test_decode_once_matches_oracle_and_tile_kernel(gpu, mats, xs, name):
    import torch
    m, W_hat = mats[name]
    g = m.device_tiles(gpu)
    Xf, Xb = xs
    assert g.lib.mtc_set_prefill_decode_once(-1) == 1
    fmt = ("gathered columns" if g.desc.flags & _abi.MTC_FLAG_COLS_GATHERED else
           "fp32 scales" if g.desc.flags & _abi.MTC_FLAG_FP32_SCALES else "bf16 scales")
    _say("decode-once", name, fmt, "row_perm" if g.host.row_perm is not None else "")
    Y = g.gemm_bf16(Xb)
    torch.cuda.synchronize()
    # the decoded weight sits at the start of the workspace: Wt[n][k] = bf16(W_hat[row_perm[k], n])
    ws, _ = g.workspace(M, 1)
    ldw = 64 * g.host.n_ksteps
    Wt = ws[: N * ldw * 2].view(torch.bfloat16).view(N, ldw)[:, :K].float().cpu().numpy()
    rows = g.host.row_perm if g.host.row_perm is not None else np.arange(K)
    want = O.bf16_round(W_hat[rows]).T + np.float32(0.0)
    assert np.array_equal(_bits(Wt), _bits(want)), name
    Y = Y.cpu().numpy()
    err = O.relative_frobenius_error(O.qt_gemm_f64(Xb.float().cpu().numpy(), W_hat), Y)
    assert err <= TOL_BF16, (name, err)
    assert np.array_equal(_bits(g.gemm_bf16(Xb).cpu().numpy()), _bits(Y)), "repeat"
    Yt = _fused(lambda: g.gemm_bf16(Xb)).cpu().numpy()
    assert O.relative_frobenius_error(Yt, Y) <= 1e-5, name
    # fp32 X is staged to bf16 first: the same GEMM on the same operands
    assert np.array_equal(_bits(g.gemm_bf16(Xf).cpu().numpy()), _bits(Y)), "fp32 X"


def test_decode_once_bf16_output_and_strided_x(gpu, mats, xs):
    import torch
    m, W_hat = mats["qt"]
    g = m.device_tiles(gpu)
    _, Xb = xs
    _say("decode-once bf16 Y, strided X")
    ref = O.qt_gemm_f64(Xb.float().cpu().numpy(), W_hat)
    Yb = g.gemm_bf16(Xb, out_dtype=torch.bfloat16).float().cpu().numpy()
    assert O.relative_frobenius_error(ref, Yb) <= TOL_BF16 + 4e-3
    big = torch.zeros(M, K + 64, device=gpu, dtype=torch.bfloat16)
    big[:, :K] = Xb
    Ys = g.gemm_bf16(big[:, :K]).cpu().numpy()
    assert O.relative_frobenius_error(ref, Ys) <= TOL_BF16


def _col_permuted_tiles(gpu, N_, seed):
    """A QT-P matrix packed with its column permutation kept (bf16-pair cells and col_perm, not
    gathered columns): the tile kernel at every M, since a GEMM cannot scatter Y's columns."""
    from tensorpack_amd.device import DeviceTiles
    from tensorpack_amd.tilestream import pack_tiles
    Wn = outlier_matrix(seed, K, N_)
    a = PermutedQuadtreeRD(Wn, None, (32, 16, 8, 4)).select(4.5)
    lv = MTCMatrix.from_quadtree(a, Wn)._levels
    ts = pack_tiles(lv.shape, lv.sizes, lv.leaf, lv.modes, lv.scales, lv.codes_of, lv.scale_format, lv.row_perm,
                    lv.col_perm, gather_cols=False)
    assert ts.col_perm is not None
    return DeviceTiles(ts, gpu)


def test_decode_once_group_members_equal_single_calls(gpu, mats, xs):
    """A group of an eligible member and one that runs the tile kernel (a column permutation,
    N = 256: 16 tiles, split K): each Y equals its single call bit for bit."""
    from tensorpack_amd.device import gemm_bf16_group
    small = _col_permuted_tiles(gpu, 256, 74)
    g = mats["qt"][0].device_tiles(gpu)
    _, Xb = xs
    for X in (Xb, Xb.float()):
        _say("decode-once group", X.dtype)
        Ys = gemm_bf16_group([small, g], X)
        assert np.array_equal(_bits(Ys[0].cpu().numpy()), _bits(small.gemm_bf16(X).cpu().numpy()))
        assert np.array_equal(_bits(Ys[1].cpu().numpy()), _bits(g.gemm_bf16(X).cpu().numpy()))


@pytest.mark.parametrize("Mb", [512, 600])
def test_decode_once_batch_members_equal_single_calls(gpu, mats, Mb):
    """A batch that does not fill the chip (an eligible member from 512 rows on, and a column-
    permuted one on the tile kernel): each member's Y equals its single call bit for bit, the
    eligible one on the decode-once path; relaunching gives the same bits."""
    import torch
    from tensorpack_amd.device import GemmBatch
    g = mats["qt"][0].device_tiles(gpu)
    small = _col_permuted_tiles(gpu, 256, 75)
    rng = np.random.RandomState(Mb)
    Xs = [torch.from_numpy(rng.randn(Mb, K).astype(np.float32)).to(gpu).to(torch.bfloat16) for _ in range(2)]
    _say("decode-once batch", Mb)
    b = GemmBatch([g, small], Xs)
    ys = [y.clone() for y in b.launch()]
    torch.cuda.synchronize()
    assert np.array_equal(_bits(ys[0].cpu().numpy()), _bits(g.gemm_bf16(Xs[0]).cpu().numpy()))
    assert np.array_equal(_bits(ys[1].cpu().numpy()), _bits(small.gemm_bf16(Xs[1]).cpu().numpy()))
    b.launch()
    torch.cuda.synchronize()
    for y0, y in zip(ys, b.outs):
        assert torch.equal(y0, y)
    # the plan keeps the path it was built with, whatever the switch says at launch
    _fused(lambda: b.launch())
    torch.cuda.synchronize()
    for y0, y in zip(ys, b.outs):
        assert torch.equal(y0, y)


def _capture(fn, out, reps=3):
    """Capture fn() (writing `out`) into a HIP graph on a side stream and replay it `reps` times,
    with eager work and a synchronisation between replays; returns each replay's output."""
    import torch
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    res = []
    for _ in range(reps):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        res.append(out.clone())
    return res


def _first_call_under_capture(fn, out, eager_fn, tol):
    """A shape's first call made while a graph is captured. If nothing has set up the library in
    this process outside a capture, the graph holds the tile kernel (the library is never set up
    during a capture); either way its replays agree with each other, and with the eager call within
    `tol`. A second capture, after the eager call, equals the eager call bit for bit."""
    import torch
    first = _capture(fn, out)
    eager = eager_fn()
    torch.cuda.synchronize()
    for r in first[1:]:
        assert torch.equal(r, first[0])
    assert O.relative_frobenius_error(eager.cpu().numpy(), first[0].cpu().numpy()) <= tol
    for r in _capture(fn, out):
        assert torch.equal(r, eager)


def test_decode_once_first_call_under_graph_capture(gpu, mats):
    import torch
    g = mats["uniform"][0].device_tiles(gpu)
    X = torch.from_numpy(np.random.RandomState(76).randn(700, K).astype(np.float32)).to(gpu).to(torch.bfloat16)
    out = torch.empty(700, N, device=gpu)
    _say("decode-once first call under capture")
    _first_call_under_capture(lambda: g.gemm_bf16(X, out=out), out, lambda: g.gemm_bf16(X), 1e-5)


def test_decode_once_f32_first_call_under_graph_capture(gpu, mats):
    import torch
    g = mats["qtp"][0].device_tiles(gpu)
    M_ = 1100                                          # 1100 x 1024 x 4096 >= 2^32: the fp32 path
    X = torch.from_numpy(np.random.RandomState(95).randn(M_, K).astype(np.float32)).to(gpu)
    out = torch.empty(M_, N, device=gpu)
    _say("decode-once fp32 first call under capture")
    _first_call_under_capture(lambda: g.gemm_f32(X, out=out), out, lambda: g.gemm_f32(X), 1e-6)


@pytest.mark.parametrize("K_,N_,M_", [(992, 544, 1024), (96, 4096, 1024), (2048, 288, 600)])
def test_decode_once_ragged_shapes(gpu, K_, N_, M_):
    """K not a multiple of 64 (the decoded rows past K hold the stream's zero padding and the GEMM
    reads K of them), N not a multiple of 256 (the last column tile decodes columns past N that
    are not written) and M not a multiple of any tile height: Y within the bf16 bar of the fp64
    product, the decoded W_hat bit-exact in the workspace, the tile kernel's Y within 1e-5."""
    import torch
    W = outlier_matrix(K_ + N_, K_, N_)
    a = QuadtreeRD(W, None, (32, 16, 8, 4)).select(4.5)
    W_hat = O.qt_dequant(W, a.sizes, a.leaf, a.modes, a.scales)
    g = MTCMatrix.from_quadtree(a, W).device_tiles(gpu)
    assert M_ * K_ * N_ >= 1 << 28 and M_ >= max(512, K_ // 8)          # eligible
    X = torch.from_numpy(np.random.RandomState(K_).randn(M_, K_).astype(np.float32)).to(gpu).to(torch.bfloat16)
    _say("decode-once ragged", K_, N_, M_)
    Y = g.gemm_bf16(X)
    torch.cuda.synchronize()
    ws, _ = g.workspace(M_, 1)
    ldw = 64 * g.host.n_ksteps
    Wt = ws[: N_ * ldw * 2].view(torch.bfloat16).view(N_, ldw).float().cpu().numpy()
    assert np.array_equal(_bits(Wt[:, :K_]), _bits(O.bf16_round(W_hat).T + np.float32(0.0)))
    assert not Wt[:, K_:].any()
    Y = Y.cpu().numpy()
    assert O.relative_frobenius_error(O.qt_gemm_f64(X.float().cpu().numpy(), W_hat), Y) <= TOL_BF16
    assert O.relative_frobenius_error(_fused(lambda: g.gemm_bf16(X)).cpu().numpy(), Y) <= 1e-5


@pytest.mark.parametrize("name", ["qt", "qtp", "uniform"])
def test_decode_once_f32(gpu, mats, xs, name):
    """fp32 results (mtc_gemm_f32) from 256 rows and 2^32 multiply-adds on: the exact W_hat decoded
    once into fp32 (bit-exact against the oracle in the stream's row order) and hipBLASLt's fp32
    GEMM; Y within the fp32 bar (1e-5) of the fp64 product and within 1e-6 of the fp32 tile
    kernel's Y; repeated calls bit-identical."""
    import torch
    m, W_hat = mats[name]
    g = m.device_tiles(gpu)
    Xf, _ = xs
    X = Xf[:1024]
    _say("decode-once fp32", name)
    Y = g.gemm_f32(X)
    torch.cuda.synchronize()
    ws, _ = g.workspace(1024, 0, int(g.lib.mtc_gemm_f32_workspace_bytes(ctypes.byref(g.desc), 1024)))
    ldw = 64 * g.host.n_ksteps
    Wt = ws[: N * ldw * 4].view(torch.float32).view(N, ldw)[:, :K].cpu().numpy()
    rows = g.host.row_perm if g.host.row_perm is not None else np.arange(K)
    assert np.array_equal(_bits(Wt), _bits(W_hat[rows].T + np.float32(0.0))), name
    Y = Y.cpu().numpy()
    err = O.relative_frobenius_error(O.qt_gemm_f64(X.cpu().numpy(), W_hat), Y)
    assert err <= 1e-5, (name, err)
    assert np.array_equal(_bits(g.gemm_f32(X).cpu().numpy()), _bits(Y)), "repeat"
    Yt = _fused(lambda: g.gemm_f32(X)).cpu().numpy()
    assert O.relative_frobenius_error(Yt, Y) <= 1e-6, name


def test_decode_once_two_threads_two_streams(gpu, mats):
    """Two host threads, each on its own HIP stream, make the first calls of new shapes at the same
    time (plans made concurrently; one prefill workspace per stream): each Y equals the same call
    made alone afterwards, bit for bit."""
    import threading
    import torch
    tiles = [mats["qt"][0].device_tiles(gpu), mats["qtp"][0].device_tiles(gpu)]
    Ms = (900, 1100)
    Xs = [torch.from_numpy(np.random.RandomState(90 + i).randn(M_, K).astype(np.float32)).to(gpu).to(torch.bfloat16)
          for i, M_ in enumerate(Ms)]
    outs, errs = [None, None], []

    def run(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for _ in range(3):
                    outs[i] = tiles[i].gemm_bf16(Xs[i])
            s.synchronize()
        except Exception as ex:            # reported below, in the test's own thread
            errs.append(ex)

    _say("decode-once two threads")
    th = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert not errs, errs
    for i in range(2):
        assert torch.equal(outs[i], tiles[i].gemm_bf16(Xs[i])), i

