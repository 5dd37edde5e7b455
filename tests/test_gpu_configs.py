"""GPU parity at the five benchmark workloads' full sizes (tensorpack_amd.workloads c1-c5).

Every case builds its workload's seeded weights and allocation exactly as bench.py does,
runs the HIP path in the layout the benchmark uses, and checks it against the oracle
(the reference's bars, tests/test_allocation.py:69-86 and tests/test_permutation.py:38-50):

- W_hat through k_dequant bit-exact to the oracle's qt_dequant / permuted_qt_dequant;
- fp32 decode path: Y within relative Frobenius 1e-5 of the fp64 product X @ W_hat;
- bf16 MFMA path: Y within 2e-3 of the fp64 product bf16(X) @ W_hat.

c1: 1024^2 QT @ 3.125, M = 64 (fp32 and bf16 paths); c2: 4096^2 QT-P @ 4.25, M = 1 and 16
in the bench's decode layout (one 4096-row chunk, X rows gathered on chip); c3: one
Qwen2.5-0.5B-shaped layer (q, k, v, o, gate, up, down), QT-P @ 3.125, M = 1 (the 4864-row
down projection in 5 row chunks with the cross-block reduction) and M = 512 (split K),
single and grouped launches; c4: 8192^2 QT @ 4.5 at M = 4096 bf16 (16 x 32 output tiles,
no split), 64 sampled rows covering every row tile and every column tile; c5: the
adversarial leaf mix @ 2.5, M = 1 and M = 256.
"""

import numpy as np
import pytest

from oracle import mtc_oracle as O
from tensorpack_amd import workloads
from tensorpack_amd.kernels.gemm import MTCMatrix, mtc_gemm, mtc_gemm_group

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5
TOL_BF16 = 2e-3


def _say(*a):
    print("[configs]", *a, flush=True)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _oracle_what(alloc, W):
    if hasattr(alloc, "inner"):
        i = alloc.inner
        return O.permuted_qt_dequant(W, alloc.row_perm, alloc.col_perm, i.sizes, i.leaf, i.modes, i.scales)
    return O.qt_dequant(W, alloc.sizes, alloc.leaf, alloc.modes, alloc.scales)


_CACHE = {}


def _workload(name):
    """(workload, allocation, packed matrix, oracle W_hat) of a single-matrix config, built once."""
    if name not in _CACHE:
        wl = workloads.CONFIGS[name]()
        _say(name, "allocating", wl.W.shape, "@", wl.budget)
        a = wl.allocate()
        _CACHE[name] = (wl, a, MTCMatrix.from_quadtree(a, wl.W), _oracle_what(a, wl.W))
    return _CACHE[name]


def _check_dequant(name, m, W_hat):
    _say(name, "k_dequant", m.shape)
    got = m.to_array()
    assert np.array_equal(_bits(got), _bits(W_hat)), name
    del got


def _check_f32(name, X, Y, W_hat):
    Y = Y.cpu().numpy() if hasattr(Y, "cpu") else Y
    err = O.relative_frobenius_error(O.qt_gemm_f64(X, W_hat), Y)
    _say(name, f"fp32 path rel {err:.2e}")
    assert err < TOL_F32, (name, err)


def _check_bf16(name, X, Y, W_hat):
    Y = Y.float().cpu().numpy() if hasattr(Y, "cpu") else Y
    err = O.relative_frobenius_error(O.qt_gemm_f64(O.bf16_round(X), W_hat), Y)
    _say(name, f"bf16 path rel {err:.2e}")
    assert err < TOL_BF16, (name, err)


def test_c1_m64(gpu):
    import torch
    wl, a, m, W_hat = _workload("c1")
    _check_dequant("c1", m, W_hat)
    X = wl.activations(64)
    _say("c1 M=64 fp32 decode")
    _check_f32("c1 M=64", X, mtc_gemm(torch.from_numpy(X).to(gpu), m, compute="fp32"), W_hat)
    _say("c1 M=64 bf16 prefill")
    _check_bf16("c1 M=64", X, mtc_gemm(torch.from_numpy(X).to(gpu), m), W_hat)


@pytest.mark.parametrize("M", [1, 16])
def test_c2_decode(gpu, M):
    import torch
    wl, a, m, W_hat = _workload("c2")
    if M == 1:
        _check_dequant("c2", m, W_hat)
    ds = m.device_stream(None, gpu, M)              # the bench's decode layout
    # M = 1: whole 4096-row units; M = 16 (matrix core, 16-row M tile): 2048-row units, split K
    assert ds.host.chunk_rows == (4096 if M == 1 else 2048) and ds.host.row_perm is not None
    X = wl.activations(M)
    _say(f"c2 M={M} decode, chunk_rows {ds.host.chunk_rows}")
    Y = ds.gemv_f32(torch.from_numpy(X).to(gpu))
    _check_f32(f"c2 M={M}", X, Y, W_hat)
    Y2 = mtc_gemm(torch.from_numpy(X).to(gpu), m)
    assert torch.equal(Y, Y2)
    if M == 16:                                     # the fp32 matrix-core tile path at the same rows
        _check_f32(f"c2 M={M} (fp32 tiles)", X, m.device_tiles(gpu).gemm_f32(torch.from_numpy(X).to(gpu)), W_hat)
    if M == 16:                                     # the M = 1 layout at M = 16: two 8-row M tiles
        _say("c2 M=16 decode, chunk_rows 4096")
        _check_f32("c2 M=16 (4096-row units)", X, m.device_stream(4096, gpu).gemv_f32(torch.from_numpy(X).to(gpu)),
                   W_hat)


def test_c4_prefill(gpu):
    import torch
    wl, a, m, W_hat = _workload("c4")
    _check_dequant("c4", m, W_hat)
    M = 4096
    X = torch.from_numpy(wl.activations(M)).to(gpu).to(torch.bfloat16)
    t = m.device_tiles(gpu)
    assert t.host.n_col_tiles == 32 and t.host.n_ksteps == 128
    from tensorpack_amd._abi import MTC_DTYPE_BF16
    from tensorpack_amd.device import set_prefill_decode_once
    ws, nbytes = t.workspace(M, MTC_DTYPE_BF16)
    # the decode-once path: W_hat in bf16, no staging (bf16 X read in place), no GEMM workspace
    assert nbytes == 8192 * 8192 * 2
    rng = np.random.RandomState(4242)
    rows = np.concatenate([rt * 256 + np.r_[0, 255, rng.choice(np.arange(1, 255), 2, replace=False)]
                           for rt in range(16)])
    Xs = X[torch.from_numpy(rows).to(gpu)].float().cpu().numpy()      # exact bf16 values
    ref = O.qt_gemm_f64(Xs, W_hat)
    for once in (True, False):                       # the library's choice, then the fused tile kernel
        _say("c4 M=4096 prefill", "decode once + GEMM" if once else "tile kernel")
        prev = set_prefill_decode_once(once)
        try:
            Y = t.gemm_bf16(X)
            torch.cuda.synchronize()
        finally:
            set_prefill_decode_once(prev)
        Ys = Y[torch.from_numpy(rows).to(gpu)].cpu().numpy()
        err = O.relative_frobenius_error(ref, Ys)
        _say(f"c4 M=4096 sampled {rows.size} rows rel {err:.2e}")
        assert err < TOL_BF16
        for ct in range(32):                             # each column tile on its own
            sl = slice(256 * ct, 256 * ct + 256)
            assert O.relative_frobenius_error(ref[:, sl], Ys[:, sl]) < TOL_BF16, ct
        for rt in range(16):                             # each row tile on its own
            sl = slice(4 * rt, 4 * rt + 4)
            assert O.relative_frobenius_error(ref[sl], Ys[sl]) < TOL_BF16, rt
        assert torch.isfinite(Y).all()


@pytest.mark.parametrize("M", [1, 256])
def test_c5(gpu, M):
    import torch
    wl, a, m, W_hat = _workload("c5")
    if M == 1:
        _check_dequant("c5", m, W_hat)
    X = wl.activations(M)
    _say(f"c5 M={M}")
    Y = mtc_gemm(torch.from_numpy(X).to(gpu), m)
    (_check_f32 if M <= 16 else _check_bf16)(f"c5 M={M}", X, Y, W_hat)


@pytest.fixture(scope="module")
def c3_layer():
    mats = workloads.c3_matrices(1)
    _say("c3 layer 0: allocating", len(mats), "matrices")
    allocs = [w.allocate() for w in mats]
    return [(w, a, MTCMatrix.from_quadtree(a, w.W), _oracle_what(a, w.W)) for w, a in zip(mats, allocs)]


def test_c3_layer_dequant(gpu, c3_layer):
    for w, a, m, W_hat in c3_layer:
        _check_dequant(w.name, m, W_hat)


def test_c3_layer_m1(gpu, c3_layer):
    import torch
    outs = {}
    for w, a, m, W_hat in c3_layer:
        ds = m.device_stream(None, gpu, 1)
        if w.W.shape == (4864, 896):                 # the down projection: row chunks + cross-block sum
            assert ds.host.n_chunks == 5, ds.host.chunk_rows
        X = w.activations(1)
        _say(f"c3 {w.name} M=1 (chunks {ds.host.n_chunks})")
        Y = mtc_gemm(torch.from_numpy(X).to(gpu), m)
        _check_f32(w.name + " M=1", X, Y, W_hat)
        Y2 = mtc_gemm(torch.from_numpy(X).to(gpu), m)
        assert torch.equal(Y, Y2)                    # the split-K reduction is deterministic
        outs[w.name] = Y
    # q/k/v and gate/up read one input each: grouped launches, bit-identical to single calls
    for members in ((0, 1, 2), (4, 5)):
        w0 = c3_layer[members[0]][0]
        X = torch.from_numpy(w0.activations(1)).to(gpu)
        _say("c3 M=1 group", [c3_layer[i][0].name for i in members])
        ys = mtc_gemm_group(X, [c3_layer[i][2] for i in members])
        for i, y in zip(members, ys):
            w, a, m, W_hat = c3_layer[i]
            assert torch.equal(y, mtc_gemm(X, m)), w.name
            _check_f32(w.name + " M=1 grouped", w0.activations(1), y, W_hat)


def test_c3_layer_m512(gpu, c3_layer):
    import torch
    from tensorpack_amd._abi import MTC_DTYPE_F32
    M = 512
    for w, a, m, W_hat in c3_layer:
        t = m.device_tiles(gpu)
        if w.W.shape == (4864, 896) or w.W.shape == (896, 896):
            ws, nbytes = t.workspace(M, MTC_DTYPE_F32)
            assert nbytes > M * w.W.shape[0] * 2 + 256, w.name   # split-K partials beyond the staged X
        X = w.activations(M)
        _say(f"c3 {w.name} M=512 prefill")
        Y = mtc_gemm(torch.from_numpy(X).to(gpu), m)
        _check_bf16(w.name + " M=512", X, Y, W_hat)
    for members in ((0, 1, 2), (4, 5)):
        w0 = c3_layer[members[0]][0]
        X = torch.from_numpy(w0.activations(M)).to(gpu)
        _say("c3 M=512 group", [c3_layer[i][0].name for i in members])
        ys = mtc_gemm_group(X, [c3_layer[i][2] for i in members])
        for i, y in zip(members, ys):
            w, a, m, W_hat = c3_layer[i]
            assert torch.equal(y, mtc_gemm(X, m)), w.name
            _check_bf16(w.name + " M=512 grouped", w0.activations(M), y, W_hat)
