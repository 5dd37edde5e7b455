"""Channel-permuted quadtree allocation (rows and columns sorted before the tree).

Restates mtc/core/permutation.py:34-105. Rows (input channels) are sorted by
h_k * ||W_k,:||^2 and columns by sum_k h_k W_kj^2 (stable argsort, ascending);
the quadtree then runs on Wp = W[pr][:, pc] with h[pr]. The index arrays are
stored data and are charged ceil(log2 K) bits per row index and ceil(log2 N)
per column index.

Inference identity (permutation.py:15-18): Y[:, pc] = X[:, pr] @ Wp_hat.
The GPU kernels fold the pr gather into their X loads and the pc scatter into
their Y stores.
"""

from math import ceil, log2
from typing import Optional, Sequence, Tuple

import numpy as np

from .allocation import DEFAULT_MODES
from .quadtree import QTAllocation, QuadtreeRD, qt_dequant


def channel_orders(W: np.ndarray, importance: Optional[np.ndarray], rows: bool = True,
                   cols: bool = True) -> Tuple[np.ndarray, np.ndarray]:
    K, N = W.shape
    h = np.ones(K) if importance is None else np.asarray(importance, dtype=np.float64)
    energy = h[:, None] * (np.asarray(W, dtype=np.float64) ** 2)
    pr = np.argsort(energy.sum(axis=1), kind="stable") if rows else np.arange(K)
    pc = np.argsort(energy.sum(axis=0), kind="stable") if cols else np.arange(N)
    return pr, pc


def index_bits(K: int, N: int, rows: bool, cols: bool) -> int:
    """Bits to store the permutations; identity orders are not stored."""
    return (K * ceil(log2(K)) if rows else 0) + (N * ceil(log2(N)) if cols else 0)


def unpermute(Wp: np.ndarray, pr: np.ndarray, pc: np.ndarray) -> np.ndarray:
    out = np.empty_like(Wp)
    out[np.ix_(pr, pc)] = Wp
    return out


def permuted_qt_dequant(W: np.ndarray, pr, pc, sizes, leaf, modes, scales) -> np.ndarray:
    Wp = np.asarray(W, dtype=np.float32)[pr][:, pc]
    return unpermute(qt_dequant(Wp, sizes, leaf, modes, scales), pr, pc)


class PermutedQTAllocation:
    """Inner quadtree allocation of Wp plus the two orders (permutation.py:54-67)."""

    def __init__(self, inner: QTAllocation, row_perm: np.ndarray, col_perm: np.ndarray, total_bits: int,
                 dequant: Optional[np.ndarray] = None):
        self.inner = inner
        self.row_perm = row_perm
        self.col_perm = col_perm
        self.total_bits = int(total_bits)
        self._dequant = dequant

    @property
    def shape(self):
        return self.inner.shape

    @property
    def dequant(self) -> np.ndarray:
        """W_hat in the ORIGINAL channel order."""
        if self._dequant is None:
            self._dequant = unpermute(self.inner.dequant, self.row_perm, self.col_perm)
        return self._dequant

    @property
    def bits_per_element(self) -> float:
        return self.total_bits / (self.shape[0] * self.shape[1])

    def leaf_area_fraction(self):
        return self.inner.leaf_area_fraction()


class PermutedQuadtreeRD:
    """Same budgets as QuadtreeRD, with the permutation index bits charged."""

    def __init__(self, W: np.ndarray, importance: Optional[np.ndarray] = None,
                 sizes: Sequence[int] = (32, 16, 8), modes: Sequence[int] = DEFAULT_MODES,
                 scale_format: str = "bf16", rows: bool = True, cols: bool = True, n_threads: int = 0):
        self.W = np.asarray(W, dtype=np.float32)
        h = None if importance is None else np.asarray(importance)
        self.pr, self.pc = channel_orders(self.W, h, rows, cols)
        self.perm_bits = index_bits(*self.W.shape, rows, cols)
        self.qt = QuadtreeRD(self.W[self.pr][:, self.pc], None if h is None else h[self.pr],
                             sizes, modes, scale_format, n_threads)

    def select(self, bits_per_element: float) -> PermutedQTAllocation:
        inner = self.qt.select(bits_per_element - self.perm_bits / self.W.size)
        return PermutedQTAllocation(inner, self.pr, self.pc, inner.total_bits + self.perm_bits)
