"""Batched prefill (mtc_gemm_batch_plan + mtc_gemm_bf16_batch) on the GPU.

Bars: every member's Y within 2e-3 (relative Frobenius) of the fp64 product bf16(X) @ W_hat
(plus 4e-3 for the rounding of a bf16 Y, as for single calls);
a batch too small to fill the chip splits each member's K as a single call does and then
gives the single call's Y bit for bit; members mix shapes, permutations, X dtypes per batch,
Y dtypes and split / unsplit K; relaunching is deterministic.
"""

import numpy as np
import pytest

from oracle import mtc_oracle as O
from tensorpack_amd.core.permutation import PermutedQuadtreeRD
from tensorpack_amd.core.quadtree import QuadtreeRD
from tensorpack_amd.kernels.gemm import MTCMatrix

pytestmark = pytest.mark.gpu


def _what(a, W):
    if hasattr(a, "inner"):
        i = a.inner
        return O.permuted_qt_dequant(W, a.row_perm, a.col_perm, i.sizes, i.leaf, i.modes, i.scales)
    return O.qt_dequant(W, a.sizes, a.leaf, a.modes, a.scales)


SHAPES = [  # K, N, permuted, budget
    (896, 896, True, 3.125),
    (896, 128, True, 3.125),
    (1024, 512, False, 4.5),
    (2048, 256, True, 4.25),
    (512, 1024, False, 6.0),
]


@pytest.fixture(scope="module")
def members():
    out = []
    for i, (K, N, perm, budget) in enumerate(SHAPES):
        W = (np.random.RandomState(200 + i).standard_t(4, size=(K, N)) * 0.02).astype(np.float32)
        h = np.exp(np.random.RandomState(300 + i).randn(K))
        a = (PermutedQuadtreeRD if perm else QuadtreeRD)(W, h, (32, 16, 8, 4)).select(budget)
        out.append((MTCMatrix.from_quadtree(a, W), _what(a, W)))
    return out


@pytest.mark.parametrize("M,xdt,ydt", [(96, "f32", "f32"), (300, "bf16", "f32"), (512, "f32", "bf16"),
                                       (6144, "bf16", "f32")])
def test_prefill_batch(gpu, members, M, xdt, ydt):
    import torch
    from tensorpack_amd.device import GemmBatch
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16}
    tiles = [m.device_tiles(gpu) for m, _ in members]
    rng = np.random.RandomState(M)
    Xs = [torch.from_numpy(rng.randn(M, t.K).astype(np.float32)).to(gpu).to(tdt[xdt]) for t in tiles]
    print(f"prefill batch M={M} X {xdt} Y {ydt}: plan", flush=True)
    b = GemmBatch(tiles, Xs, out_dtype=tdt[ydt])
    print("launch", flush=True)
    ys = [y.float().clone() for y in b.launch()]
    torch.cuda.synchronize()
    n_tiles = sum(-(-M // 256) * t.host.n_col_tiles for t in tiles)
    tol = 2e-3 if ydt == "f32" else 2e-3 + 4e-3      # a bf16 Y adds its own rounding (up to 2^-9 relative)
    for (m, what), t, X, y in zip(members, tiles, Xs, ys):
        Xb = X.to(torch.bfloat16).float().cpu().numpy()
        err = O.relative_frobenius_error(O.qt_gemm_f64(Xb, what), y.cpu().numpy())
        assert err < tol, (t.K, t.N, err)
        if n_tiles < 256:                     # each member splits K as its single call does
            assert torch.equal(t.gemm_bf16(X, out_dtype=tdt[ydt]).float(), y), (t.K, t.N)
    b.launch()
    torch.cuda.synchronize()
    for y0, y in zip(ys, b.outs):
        assert torch.equal(y0, y.float())
