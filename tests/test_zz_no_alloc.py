"""mtc_gemv_f32_noalloc (decode without a caller workspace; split-K scratch in a static
per-device array) called through the C-ABI, against mtc_gemv_f32 with a workspace.

Bar: bit-identical Y (same kernels, chunking and reduction order) on two calls in a row, the
second with a smaller input (fewer rows of X and a smaller matrix), for streams whose row
chunks need the cross-block reduction; oversize requests fail before any launch.
"""

import ctypes

import numpy as np
import pytest

from oracle import mtc_oracle as O
from tensorpack_amd import _abi
from tensorpack_amd.core.permutation import PermutedQuadtreeRD
from tensorpack_amd.kernels.gemm import MTCMatrix

pytestmark = pytest.mark.gpu


def _matrix(seed, K, N, budget):
    W = (np.random.RandomState(seed).standard_t(4, size=(K, N)) * 0.02).astype(np.float32)
    h = np.exp(np.random.RandomState(seed + 1).randn(K))
    a = PermutedQuadtreeRD(W, h, (32, 16, 8, 4)).select(budget)
    i = a.inner
    return MTCMatrix.from_quadtree(a, W), O.permuted_qt_dequant(W, a.row_perm, a.col_perm, i.sizes, i.leaf, i.modes,
                                                                 i.scales)


def _noalloc(ds, X, Y):
    import torch
    rc = ds.lib.mtc_gemv_f32_noalloc(ctypes.byref(ds.desc), X.data_ptr(), X.stride(0), Y.data_ptr(), Y.stride(0),
                                     X.shape[0], torch.cuda.current_stream(X.device).cuda_stream)
    _abi.check(ds.lib, "mtc_gemv_f32_noalloc", rc)


def test_noalloc_matches_workspace_path(gpu):
    import torch
    big, big_hat = _matrix(81, 4864, 896, 3.125)      # the decode layout splits K into 5 row chunks
    small, small_hat = _matrix(82, 1024, 256, 4.25)
    calls = [(big, big_hat, 16, None), (small, small_hat, 3, 256)]   # second call: smaller M and matrix
    for m, what, M, cr in calls:
        ds = m.device_stream(cr, gpu, M)
        assert ds.host.n_chunks > 1
        X = torch.randn(M, ds.K, device=gpu)
        print(f"noalloc: K={ds.K} N={ds.N} M={M} chunks={ds.host.n_chunks}", flush=True)
        ref = ds.gemv_f32(X)
        Y = torch.full((M, ds.N), float("nan"), device=gpu)
        _noalloc(ds, X, Y)
        torch.cuda.synchronize()
        assert torch.equal(Y, ref)
        err = O.relative_frobenius_error(O.qt_gemm_f64(X.cpu().numpy(), what), Y.cpu().numpy())
        assert err < 1e-5, err
    # the same stream again after the other one used the scratch (counters cleared per call)
    ds = big.device_stream(None, gpu, 16)
    X = torch.randn(16, ds.K, device=gpu)
    Y = torch.empty(16, ds.N, device=gpu)
    _noalloc(ds, X, Y)
    torch.cuda.synchronize()
    assert torch.equal(Y, ds.gemv_f32(X))


def test_noalloc_rejects_oversize_before_launch(gpu):
    import torch
    m, _ = _matrix(83, 4096, 4096, 4.25)
    ds = m.device_stream(512, gpu, 16)                 # 8 row chunks
    lib = ds.lib
    cap = lib.mtc_gemv_noalloc_scratch_bytes()
    assert cap == 8 << 20
    M = 4096                                           # 1024 M tiles x 128 panels x 8 chunks x 4 rows x 32 x 4 B
    assert lib.mtc_gemv_workspace_bytes(ctypes.byref(ds.desc), M) > cap
    X = torch.zeros(M, ds.K, device=gpu)
    Y = torch.zeros(M, ds.N, device=gpu)
    rc = lib.mtc_gemv_f32_noalloc(ctypes.byref(ds.desc), X.data_ptr(), ds.K, Y.data_ptr(), ds.N, M, None)
    assert rc == -5 and b"scratch" in lib.mtc_last_error()
    torch.cuda.synchronize()
    assert not Y.any()
