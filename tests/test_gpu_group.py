"""GPU parity of the grouped decode launch (mtc_gemv_f32_group) and the linear layers.

Bars: every member's Y is bit-identical to its own mtc_gemm call (the grouped kernel runs
the same block code on the same data), and within relative Frobenius 1e-5 of the fp64
oracle X @ W_hat (the fp32-path bar). Layer outputs add the bias in fp32.
"""

import numpy as np
import pytest

from oracle import mtc_oracle as O
from tensorpack_amd import _abi
from tensorpack_amd.core.permutation import PermutedQuadtreeRD
from tensorpack_amd.core.quadtree import QuadtreeRD
from tensorpack_amd.kernels.gemm import MTCMatrix, mtc_gemm, mtc_gemm_group
from tensorpack_amd.nn import LinearMTC, LinearMTCGroup, seeded_fp32_weight

from conftest import outlier_matrix

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5

# a decoder layer in miniature: q, k, v (QT-P, shared K) plus an unpermuted member
MEMBERS = [("q", 256, 256, True, 3.125), ("k", 256, 64, True, 3.125), ("v", 256, 64, True, 3.125),
           ("wide", 256, 384, True, 4.25), ("plain", 256, 96, False, 2.5)]


def _say(*a):
    print(*a, flush=True)


def _oracle_what(alloc, W):
    if hasattr(alloc, "inner"):
        i = alloc.inner
        return O.permuted_qt_dequant(W, alloc.row_perm, alloc.col_perm, i.sizes, i.leaf, i.modes, i.scales)
    return O.qt_dequant(W, alloc.sizes, alloc.leaf, alloc.modes, alloc.scales)


@pytest.fixture(scope="module")
def members():
    out = []
    for j, (name, K, N, perm, budget) in enumerate(MEMBERS):
        W = outlier_matrix(40 + j, K, N)
        h = np.exp(np.random.RandomState(140 + j).randn(K))
        a = (PermutedQuadtreeRD if perm else QuadtreeRD)(W, h, (32, 16, 8, 4)).select(budget)
        out.append((name, W, a, MTCMatrix.from_quadtree(a, W)))
    return out


@pytest.mark.parametrize("M", [1, 2, 3, 5, 16])
@pytest.mark.parametrize("pick", [(0, 1, 2), (0, 1, 2, 3), (0, 1, 2, 3, 4), (4,), (3, 0)])
def test_group_matches_single_calls_bit_for_bit(gpu, members, M, pick):
    import torch
    _say("group", pick, M)
    X = np.random.RandomState(M + 10 * len(pick)).randn(M, 256).astype(np.float32)
    Xd = torch.from_numpy(X).to(gpu)
    mats = [members[i][3] for i in pick]
    ys = mtc_gemm_group(Xd, mats)
    torch.cuda.synchronize()
    assert len(ys) == len(pick)
    for i, y in zip(pick, ys):
        name, W, a, m = members[i]
        single = mtc_gemm(Xd, m, compute="fp32")
        assert torch.equal(y, single), (name, M)
        err = O.relative_frobenius_error(O.qt_gemm_f64(X, _oracle_what(a, W)), y.cpu().numpy())
        assert err <= TOL_F32, (name, M, err)


def test_group_numpy_vector_and_strided_outputs(gpu, members):
    import torch
    from tensorpack_amd.device import gemv_f32_group
    _say("group numpy / vector / strided")
    x = np.random.RandomState(5).randn(256).astype(np.float32)
    ys = mtc_gemm_group(x, [members[0][3], members[1][3]])
    assert all(isinstance(y, np.ndarray) and y.shape == (members[i][3].shape[1],) for i, y in enumerate(ys))
    for (name, W, a, m), y in zip(members[:2], ys):
        assert np.array_equal(y, mtc_gemm(x, m)), name
    # outputs that are column slices of one wide buffer (leading dimension > N)
    X = torch.from_numpy(np.random.RandomState(6).randn(3, 256).astype(np.float32)).to(gpu)
    big = torch.full((3, 256 + 64 + 64), float("nan"), device=gpu)
    outs = [big[:, :256], big[:, 256:320], big[:, 320:]]
    streams = [members[i][3].device_stream(None, gpu, 3) for i in range(3)]
    gemv_f32_group(streams, X, outs)
    torch.cuda.synchronize()
    for (name, W, a, m), o in zip(members[:3], outs):
        assert torch.equal(o, mtc_gemm(X, m, compute="fp32")), name


def test_group_rejects_split_k_streams(gpu, members):
    import torch
    from tensorpack_amd.device import gemv_f32_group
    _say("group split-K rejection")
    m = members[0][3]
    X = torch.zeros((1, 256), device=gpu)
    with pytest.raises(_abi.MtcError):
        gemv_f32_group([m.device_stream(64, gpu)], X)                 # four row chunks
    with pytest.raises(ValueError):
        gemv_f32_group([m.device_stream(None, gpu)] * (_abi.MAX_GROUP + 1), X)


@pytest.mark.parametrize("M", [1, 4, 40])
def test_linear_layers(gpu, M):
    import torch
    _say("linear layers", M)
    rng = np.random.RandomState(M)
    q = LinearMTC(256, 128, budget_bits=4.0, seed=7, bias=rng.randn(128).astype(np.float32))
    k = LinearMTC(256, 64, budget_bits=3.0, seed=8, permuted=False)
    X = rng.randn(M, 256).astype(np.float32)
    for lin, seed in ((q, 7), (k, 8)):
        what = _oracle_what(lin.alloc, seeded_fp32_weight(256, lin.out_features, seed))
        # above 16 rows the bf16 MFMA path runs: its reference takes the same bf16-rounded X
        Xr = X if M <= 16 else torch.from_numpy(X).bfloat16().float().numpy()
        ref = O.qt_gemm_f64(Xr, what) + lin.b.astype(np.float64)
        tol = TOL_F32 if M <= 16 else 2e-3
        y = lin(X)
        assert isinstance(y, np.ndarray) and y.shape == (M, lin.out_features)
        assert O.relative_frobenius_error(ref, y) <= tol
        yd = lin(torch.from_numpy(X).to(gpu))
        assert isinstance(yd, torch.Tensor) and yd.device.type == "cuda"
        assert np.array_equal(yd.cpu().numpy(), y)
    g = LinearMTCGroup([q, k])
    ys = g(torch.from_numpy(X).to(gpu))
    for lin, y in zip((q, k), ys):
        assert np.array_equal(y.cpu().numpy(), lin(X)), M


@pytest.mark.parametrize("M,xdtype,ydtype", [(37, "f32", "f32"), (300, "bf16", "f32"), (600, "bf16", "bf16"),
                                             (20, "f32", "bf16")])
@pytest.mark.parametrize("pick", [(0, 1, 2), (0, 1, 2, 3, 4), (4, 3)])
def test_prefill_group_matches_single_calls_bit_for_bit(gpu, members, M, xdtype, ydtype, pick):
    import torch
    _say("prefill group", pick, M, xdtype, ydtype)
    X = np.random.RandomState(M + len(pick)).randn(M, 256).astype(np.float32)
    Xd = torch.from_numpy(X).to(gpu)
    if xdtype == "bf16":
        Xd = Xd.to(torch.bfloat16)
    odt = torch.bfloat16 if ydtype == "bf16" else torch.float32
    from tensorpack_amd.device import gemm_bf16_group
    tiles = [members[i][3].device_tiles(gpu) for i in pick]
    for j in range(0, len(tiles), _abi.MAX_GROUP):
        part = list(range(j, min(j + _abi.MAX_GROUP, len(tiles))))
        ys = gemm_bf16_group([tiles[k] for k in part], Xd, out_dtype=odt)
        torch.cuda.synchronize()
        for k, y in zip(part, ys):
            name, W, a, m = members[pick[k]]
            single = mtc_gemm(Xd, m, compute="bf16", out_dtype=odt)
            assert torch.equal(y, single), (name, M)
            ref = O.qt_gemm_f64(O.bf16_round(X), _oracle_what(a, W))
            err = O.relative_frobenius_error(ref, y.float().cpu().numpy())
            assert err <= 2e-3 + (4e-3 if ydtype == "bf16" else 0.0), (name, M, err)


def test_prefill_group_through_mtc_gemm_group(gpu, members):
    import torch
    _say("prefill group via mtc_gemm_group")
    X = torch.from_numpy(np.random.RandomState(3).randn(200, 256).astype(np.float32)).to(gpu)
    mats = [m for _, _, _, m in members]
    ys = mtc_gemm_group(X, mats)                       # 200 rows: bf16 path, 5 members -> two launches
    torch.cuda.synchronize()
    for (name, W, a, m), y in zip(members, ys):
        assert torch.equal(y, mtc_gemm(X, m)), name


def test_workspaces_are_per_stream(gpu, members):
    """Calls on two HIP streams may overlap, so each stream gets its own workspace: split-K
    decode (per-panel counters) and split-K prefill (staged X, partial tiles) interleaved on
    two streams with no synchronisation between them all match a single-stream call."""
    import torch
    _say("workspaces per stream")
    m = members[0][3]
    ds = m.device_stream(64, gpu, 2)                                  # four row chunks
    ts = m.device_tiles(gpu)
    Xd = torch.from_numpy(np.random.RandomState(9).randn(2, 256).astype(np.float32)).to(gpu)
    Xp = torch.from_numpy(np.random.RandomState(10).randn(300, 256).astype(np.float32)).to(gpu)
    ref_d, ref_p = ds.gemv_f32(Xd), ts.gemm_bf16(Xp)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)]
    outs = []
    for _ in range(10):
        for s in streams:
            with torch.cuda.stream(s):
                outs.append((ds.gemv_f32(Xd), ts.gemm_bf16(Xp)))
    torch.cuda.synchronize()
    for yd, yp in outs:
        assert torch.equal(yd, ref_d) and torch.equal(yp, ref_p)
    assert len(ds._ws) >= 2


def test_device_calls_check_their_arguments(gpu, members):
    """The launch wrappers check shapes, dtypes and devices with real exceptions (not
    asserts, which python -O removes): the kernels trust what they are given."""
    import torch
    _say("argument checks")
    m = members[0][3]
    ds, ts = m.device_stream(None, gpu, 1), m.device_tiles(gpu)
    with pytest.raises(ValueError):
        ds.gemv_f32(torch.zeros((1, 128), device=gpu))                       # K mismatch
    with pytest.raises(ValueError):
        ds.gemv_f32(torch.zeros((1, 256), device=gpu, dtype=torch.bfloat16))  # dtype
    with pytest.raises(ValueError):
        ds.gemv_f32(torch.zeros((2, 256), device=gpu), out=torch.empty((1, m.shape[1]), device=gpu))
    with pytest.raises(ValueError):
        ts.gemm_bf16(torch.zeros((40, 255), device=gpu))
    with pytest.raises(ValueError):
        ds.dequant(out=torch.empty((1, 1), device=gpu))
    from tensorpack_amd.device import require_gpu
    assert require_gpu("cuda").index is not None


@pytest.mark.parametrize("M", [1, 4])
def test_group_of_mx_streams(gpu, members, M):
    """A group in the matrix-core payload layout gives each member's own call bit for bit; a
    group may not mix layouts."""
    import torch
    from tensorpack_amd.device import gemv_f32_group
    from tensorpack_amd.packer import LAYOUT_MX
    _say("group mx", M)
    streams = [m.device_stream(None, gpu, 1, LAYOUT_MX) for _, _, _, m in members[:_abi.MAX_GROUP]]
    X = torch.from_numpy(np.random.RandomState(60 + M).randn(M, 256).astype(np.float32)).to(gpu)
    ys = gemv_f32_group(streams, X)
    torch.cuda.synchronize()
    for (name, W, a, m), s, y in zip(members, streams, ys):
        assert torch.equal(y, s.gemv_f32(X)), name
        err = O.relative_frobenius_error(O.qt_gemm_f64(X.cpu().numpy(), _oracle_what(a, W)), y.cpu().numpy())
        assert err <= TOL_F32, (name, M, err)
    with pytest.raises(_abi.MtcError):
        gemv_f32_group([streams[0], members[1][3].device_stream(None, gpu, 1)], X)
