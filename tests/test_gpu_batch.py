"""Batched decode launch (mtc_gemv_batch_plan + mtc_gemv_f32_batch) on the GPU.

Bars: every member's Y is bit-identical to its own mtc_gemv_f32 call (same block code and
chunking, fixed reduction order) and within 1e-5 of the oracle's fp64 product; members mix
shapes, permutations, row-chunk counts (split-K members with the cross-block reduction),
block record counts (8- and 16-wave blocks) and each has its own X; relaunching picks up new
X values in the same tensors; a second launch of one plan gives the same Y (the split-K
counters reset themselves).
"""

import numpy as np
import pytest

from oracle import mtc_oracle as O
from tensorpack_amd.core.permutation import PermutedQuadtreeRD
from tensorpack_amd.core.quadtree import QuadtreeRD
from tensorpack_amd.kernels.gemm import MTCMatrix

from conftest import outlier_matrix

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[batch]", *a, flush=True)


def _what(a, W):
    if hasattr(a, "inner"):
        i = a.inner
        return O.permuted_qt_dequant(W, a.row_perm, a.col_perm, i.sizes, i.leaf, i.modes, i.scales)
    return O.qt_dequant(W, a.sizes, a.leaf, a.modes, a.scales)


SHAPES = [  # K, N, permuted, budget, chunk_rows (None: the decode layout)
    (896, 896, True, 3.125, None),
    (896, 128, True, 3.125, None),
    (4864, 896, True, 3.125, None),     # 5 row chunks: split-K member
    (896, 4864, True, 3.125, None),
    (1024, 256, False, 6.0, None),
    (2048, 512, True, 4.25, 2048),      # more records per block than 16: 16-wave blocks
    (640, 96, False, 2.5, 160),         # 4 row chunks of 160 rows
]


@pytest.fixture(scope="module")
def members():
    out = []
    for i, (K, N, perm, budget, cr) in enumerate(SHAPES):
        W = (np.random.RandomState(70 + i).standard_t(4, size=(K, N)) * 0.02).astype(np.float32)
        h = np.exp(np.random.RandomState(90 + i).randn(K))
        a = (PermutedQuadtreeRD if perm else QuadtreeRD)(W, h, (32, 16, 8, 4)).select(budget)
        out.append((MTCMatrix.from_quadtree(a, W), _what(a, W), cr))
    return out


@pytest.mark.parametrize("M", [1, 2, 5, 16])
def test_batch_matches_single_calls(gpu, members, M):
    import torch
    from tensorpack_amd.device import GemvBatch
    streams = [m.device_stream(cr, gpu, M) for m, _, cr in members]
    assert any(s.host.n_chunks > 1 for s in streams) and any(s.host.fixed_steps > 16 for s in streams)
    rng = np.random.RandomState(M)
    Xs = [torch.from_numpy(rng.randn(M, s.K).astype(np.float32)).to(gpu) for s in streams]
    _say(f"M={M}: plan of {len(streams)} members")
    b = GemvBatch(streams, Xs)
    _say(f"M={M}: launch")
    ys = [y.clone() for y in b.launch()]
    torch.cuda.synchronize()
    for (m, W_hat, _), s, X, y in zip(members, streams, Xs, ys):
        ref = s.gemv_f32(X)
        assert torch.equal(y, ref), (s.K, s.N)
        err = O.relative_frobenius_error(O.qt_gemm_f64(X.cpu().numpy(), W_hat), y.cpu().numpy())
        assert err < 1e-5, (s.K, s.N, err)
    _say(f"M={M}: relaunch with new X")
    for X in Xs:
        X.copy_(torch.randn_like(X))
    b.launch()
    b.launch()
    torch.cuda.synchronize()
    for s, X, y in zip(streams, Xs, b.outs):
        assert torch.equal(y, s.gemv_f32(X)), (s.K, s.N)


@pytest.mark.parametrize("M", [3, 12])
def test_batch_strided_outputs_and_uniform_members(gpu, M):
    """fp32-scale (uniform-block) members batch together; outputs may be row-strided views."""
    import torch
    from tensorpack_amd.core.allocation import rd_allocate
    from tensorpack_amd.device import GemvBatch
    mats = []
    for i, (K, N) in enumerate(((256, 64), (512, 128), (128, 32))):
        W = outlier_matrix(40 + i, K, N)
        a = rd_allocate(W, 4.0, None, 16)
        mats.append((MTCMatrix.from_allocation(W, a.modes, a.scales, 16), a.dequant))
    streams = [m.device_stream(None, gpu, M) for m, _ in mats]
    Xs = [torch.randn(M, s.K, device=gpu) for s in streams]
    big = [torch.zeros(M, s.N + 32, device=gpu) for s in streams]
    outs = [t[:, 16:16 + s.N] for t, s in zip(big, streams)]
    _say("uniform members, strided outputs")
    GemvBatch(streams, Xs, outs).launch()
    torch.cuda.synchronize()
    for (m, what), s, X, y, t in zip(mats, streams, Xs, outs, big):
        assert torch.equal(y, s.gemv_f32(X))
        assert O.relative_frobenius_error(O.qt_gemm_f64(X.cpu().numpy(), what), y.cpu().numpy()) < 1e-5
        assert not t[:, :16].any() and not t[:, 16 + s.N:].any()


def test_batch_rejects_mixed_scale_formats(gpu, members):
    import torch
    from tensorpack_amd._abi import MtcError
    from tensorpack_amd.core.allocation import rd_allocate
    from tensorpack_amd.device import GemvBatch
    W = outlier_matrix(50, 128, 64)
    a = rd_allocate(W, 4.0, None, 16)
    uni = MTCMatrix.from_allocation(W, a.modes, a.scales, 16).device_stream(None, gpu, 1)
    qt = members[0][0].device_stream(None, gpu, 1)
    with pytest.raises(MtcError):
        GemvBatch([qt, uni], [torch.randn(1, qt.K, device=gpu), torch.randn(1, uni.K, device=gpu)])


@pytest.mark.parametrize("M", [1, 3])
def test_batch_of_mx_streams_matches_single_calls(gpu, members, M):
    """Members in the matrix-core payload layout (one X row per block) batch together and give
    their own calls' Y bit for bit, split-K members included; a batch may not mix layouts."""
    import torch
    from tensorpack_amd._abi import MtcError
    from tensorpack_amd.device import GemvBatch
    from tensorpack_amd.packer import LAYOUT_MX
    streams = [m.device_stream(cr, gpu, 1, LAYOUT_MX) for m, _, cr in members]
    assert any(s.host.n_chunks > 1 for s in streams)
    rng = np.random.RandomState(30 + M)
    Xs = [torch.from_numpy(rng.randn(M, s.K).astype(np.float32)).to(gpu) for s in streams]
    _say(f"mx M={M}: launch")
    b = GemvBatch(streams, Xs)
    b.launch()
    b.launch()
    torch.cuda.synchronize()
    for (m, W_hat, _), s, X, y in zip(members, streams, Xs, b.outs):
        assert torch.equal(y, s.gemv_f32(X)), (s.K, s.N)
        err = O.relative_frobenius_error(O.qt_gemm_f64(X.cpu().numpy(), W_hat), y.cpu().numpy())
        assert err < 1e-5, (s.K, s.N, err)
    v1 = members[0][0].device_stream(None, gpu, M)
    with pytest.raises(MtcError):
        GemvBatch([streams[0], v1], [Xs[0], Xs[0]])
