"""Linear layers over quadtree-packed weights.

`LinearMTC` is the layer the reference's `LinearMTCAdaptive` (mtc/nn/layers.py:115-151)
becomes on this path: the same construction from a seeded fp32 layer (`LinearFP32`,
mtc/nn/layers.py:67-83: W ~ U(-1/sqrt(in), 1/sqrt(in)) from RandomState(seed), zero bias),
the same `weight_bytes` / `forward` surface, but the weight is allocated by the
rate-distortion quadtree (optionally permuted) instead of the epsilon rule, and
`forward` multiplies by the packed weight on the GPU (`mtc_gemm`) instead of by a
cached dequantized copy (the reference's `X @ self._W_cached + self.b`, layers.py:150-151).

`LinearMTCGroup` runs several layers that read the same input (a decoder layer's q/k/v
or gate/up projections) through `mtc_gemm_group`: one launch per group at decode sizes.
"""

from typing import List, Optional, Sequence

import numpy as np

from .core.permutation import PermutedQuadtreeRD
from .core.quadtree import QuadtreeRD
from .kernels.gemm import MTCMatrix, mtc_gemm, mtc_gemm_group

SIZES = (32, 16, 8, 4)


def seeded_fp32_weight(in_features: int, out_features: int, seed: int = 42) -> np.ndarray:
    """The reference LinearFP32 initialisation (mtc/nn/layers.py:70-74): an (in x out) float32
    matrix drawn U(-1/sqrt(in), 1/sqrt(in)) from np.random.RandomState(seed)."""
    rng = np.random.RandomState(seed)
    std = 1.0 / np.sqrt(in_features)
    return rng.uniform(-std, std, size=(in_features, out_features)).astype(np.float32)


class LinearMTC:
    """y = x @ W_hat + b with W_hat the packed quadtree weight.

    weight      (in x out) float32; default: the reference's seeded LinearFP32 weight
    bias        (out,) float32; default zeros (as LinearFP32)
    budget_bits bits per weight for the allocator (permutation indices included when permuted)
    importance  per-input-channel weights h (default ones), e.g. mean(X_cal**2, 0)
    permuted    PermutedQuadtreeRD (True) or QuadtreeRD (False)
    """

    def __init__(self, in_features: int, out_features: int, budget_bits: float = 4.25, seed: int = 42, *,
                 weight: Optional[np.ndarray] = None, bias: Optional[np.ndarray] = None,
                 importance: Optional[np.ndarray] = None, permuted: bool = True, sizes=SIZES, n_threads: int = 0):
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        W = seeded_fp32_weight(in_features, out_features, seed) if weight is None else np.asarray(weight, np.float32)
        if W.shape != (self.in_features, self.out_features):
            raise ValueError(f"weight shape {W.shape} != ({in_features}, {out_features})")
        self.b = np.zeros(out_features, np.float32) if bias is None else np.asarray(bias, np.float32).reshape(-1)
        if self.b.shape != (self.out_features,):
            raise ValueError(f"bias shape {self.b.shape} != ({out_features},)")
        cls = PermutedQuadtreeRD if permuted else QuadtreeRD
        self.alloc = cls(W, importance, tuple(sizes), n_threads=n_threads).select(budget_bits)
        self.W_mtc = MTCMatrix.from_quadtree(self.alloc, W)
        self._bias_dev = {}

    @classmethod
    def from_matrix(cls, W_mtc: MTCMatrix, bias: Optional[np.ndarray] = None) -> "LinearMTC":
        """A layer over an already packed weight."""
        self = cls.__new__(cls)
        self.in_features, self.out_features = W_mtc.shape
        self.b = np.zeros(self.out_features, np.float32) if bias is None else np.asarray(bias, np.float32).reshape(-1)
        self.alloc = None
        self.W_mtc = W_mtc
        self._bias_dev = {}
        return self

    @property
    def weight_bytes(self) -> int:
        """Packed weight (allocator-accounted, rounded up to bytes) plus the bias, as
        LinearMTCAdaptive.weight_bytes (layers.py:147-148) counts arena bytes plus the bias."""
        return int(-(-self.W_mtc.total_bits // 8)) + self.b.nbytes

    def _add_bias(self, Y):
        if not np.any(self.b):
            return Y                                   # adding +0.0 changes nothing but the sign of -0.0
        import torch
        if isinstance(Y, torch.Tensor):
            key = (str(Y.device), Y.dtype)
            b = self._bias_dev.get(key)
            if b is None:
                b = torch.from_numpy(self.b).to(device=Y.device, dtype=Y.dtype)
                self._bias_dev[key] = b
            return Y + b
        return Y + self.b

    def forward(self, X, *, compute: str = "auto"):
        """X (M, in) or (in,), numpy or torch. numpy in -> numpy out (fp32); torch in -> device tensor."""
        return self._add_bias(mtc_gemm(X, self.W_mtc, compute=compute))

    __call__ = forward


class LinearMTCGroup:
    """Several LinearMTC layers that read the same input, run together (mtc_gemm_group)."""

    def __init__(self, layers: Sequence[LinearMTC]):
        self.layers: List[LinearMTC] = list(layers)
        if not self.layers:
            raise ValueError("empty group")
        k = self.layers[0].in_features
        if any(l.in_features != k for l in self.layers):
            raise ValueError("group members must share in_features")

    @property
    def weight_bytes(self) -> int:
        return sum(l.weight_bytes for l in self.layers)

    def forward(self, X, *, compute: str = "auto"):
        ys = mtc_gemm_group(X, [l.W_mtc for l in self.layers], compute=compute)
        return [l._add_bias(y) for l, y in zip(self.layers, ys)]

    __call__ = forward
