"""Quadtree (variable leaf size) rate-distortion allocation, offline on the CPU.

Restates mtc/core/quadtree.py:40-181. Each root tile (e.g. 32x32) is either a
leaf with its own (mode, scale) or splits into four children, down to the
finest size. For a Lagrange multiplier lambda the tree is pruned exactly,
bottom-up (quadtree.py:97-117):

    J_leaf(node) = min_mode D + lambda * (R_payload + meta)
    J(node)      = min(J_leaf(node), sum_children J(child)) + lambda * 1

(ties keep the leaf; every node above the finest level pays a 1-bit split
flag), and a 60-step bisection on log(lambda) meets the bit budget
(quadtree.py:119-154).
"""

from dataclasses import dataclass
from typing import Dict, Optional, Sequence, Tuple

import numpy as np

from .allocation import DEFAULT_MODES, RDCandidates, quantize_blocks, rd_candidates, to_blocks, from_blocks

SPLIT_FLAG_BITS = 1


def _sum4(x: np.ndarray) -> np.ndarray:
    """Children grid (2a, 2b) -> parent grid (a, b), summing each 2x2 group."""
    a, b = x.shape[0] // 2, x.shape[1] // 2
    return x.reshape(a, 2, b, 2).sum(axis=(1, 3))


def _up4(x: np.ndarray) -> np.ndarray:
    """Parent grid (a, b) -> children grid (2a, 2b), repeating each entry 2x2."""
    return np.repeat(np.repeat(x, 2, axis=0), 2, axis=1)


def qt_dequant(W: np.ndarray, sizes, leaf, modes, scales) -> np.ndarray:
    """Rebuild W_hat from W and a stored quadtree allocation (quadtree.py:157-171).

    Each level's leaves contribute q * s; levels are summed into a +0.0 buffer,
    so W_hat holds no negative zeros.
    """
    W = np.asarray(W, dtype=np.float32)
    out = np.zeros_like(W)
    for s in sizes:
        blocks = to_blocks(W, s)
        level = np.zeros_like(blocks)
        for m in np.unique(modes[s][leaf[s]]):
            if m == 0:
                continue
            sel = leaf[s] & (modes[s] == m)
            q = quantize_blocks(blocks[sel][None], int(m), scales[s][sel][None])[0]
            level[sel] = q * scales[s][sel][:, None, None]
        out += from_blocks(level)
    return out


class QTAllocation:
    """A quadtree allocation: per level s, a leaf mask, mode grid and scale grid.

    Field meaning follows quadtree.py:54-69. ``dequant`` is rebuilt lazily from
    the stored weights the first time it is read (the GPU path never needs it).
    """

    def __init__(self, sizes: Tuple[int, ...], leaf: Dict[int, np.ndarray], modes: Dict[int, np.ndarray],
                 scales: Dict[int, np.ndarray], dequant: Optional[np.ndarray], total_bits: int,
                 weights: Optional[np.ndarray] = None):
        self.sizes = tuple(sizes)
        self.leaf = leaf
        self.modes = modes
        self.scales = scales
        self.total_bits = int(total_bits)
        self._dequant = dequant
        self._weights = weights
        K = leaf[self.sizes[0]].shape[0] * self.sizes[0]
        N = leaf[self.sizes[0]].shape[1] * self.sizes[0]
        self.shape = (K, N)

    @property
    def dequant(self) -> np.ndarray:
        if self._dequant is None:
            self._dequant = qt_dequant(self._weights, self.sizes, self.leaf, self.modes, self.scales)
        return self._dequant

    @property
    def weights(self) -> Optional[np.ndarray]:
        """The (possibly permuted) float32 weights the leaves quantize."""
        return self._weights

    @property
    def bits_per_element(self) -> float:
        return self.total_bits / (self.shape[0] * self.shape[1])

    def leaf_area_fraction(self) -> Dict[int, float]:
        n = self.shape[0] * self.shape[1]
        return {s: float(self.leaf[s].sum() * s * s) / n for s in self.sizes}

    def mode_area_fraction(self) -> Dict[int, float]:
        n = self.shape[0] * self.shape[1]
        out = {int(m): 0.0 for m in DEFAULT_MODES}
        for s in self.sizes:
            for m in DEFAULT_MODES:
                out[int(m)] += float((self.leaf[s] & (self.modes[s] == m)).sum() * s * s) / n
        return out


class QuadtreeRD:
    """Candidate tables are built once per matrix; ``select(budget)`` is then cheap."""

    def __init__(self, W: np.ndarray, importance: Optional[np.ndarray] = None,
                 sizes: Sequence[int] = (32, 16, 8), modes: Sequence[int] = DEFAULT_MODES,
                 scale_format: str = "bf16", n_threads: int = 0):
        self.W = np.asarray(W, dtype=np.float32)
        self.sizes = tuple(sorted((int(s) for s in sizes), reverse=True))
        for big, small in zip(self.sizes, self.sizes[1:]):
            assert big == 2 * small, "quadtree levels must halve: e.g. (32, 16, 8)"
        K, N = self.W.shape
        assert K % self.sizes[0] == 0 and N % self.sizes[0] == 0, \
            f"shape {self.W.shape} not divisible by root size {self.sizes[0]}"
        self.cands: Dict[int, RDCandidates] = {
            s: rd_candidates(self.W, importance, s, modes, scale_format, n_threads) for s in self.sizes}

    def _solve(self, lam: float):
        """Exact tree pruning at one lambda -> (root rate grid, leaf masks, mode index grids)."""
        mode_idx, leaf_J, leaf_R = {}, {}, {}
        for s, c in self.cands.items():
            rates = c.R[:, None, None] + c.meta_bits_per_block
            J = c.D + lam * rates
            idx = np.argmin(J, axis=0)
            mode_idx[s] = idx
            leaf_J[s] = np.take_along_axis(J, idx[None], 0)[0]
            leaf_R[s] = np.take_along_axis(np.broadcast_to(rates, J.shape), idx[None], 0)[0]
        finest = self.sizes[-1]
        J, R = leaf_J[finest], leaf_R[finest]
        is_leaf = {finest: np.ones_like(J, dtype=bool)}
        for s in reversed(self.sizes[:-1]):
            split_J, split_R = _sum4(J), _sum4(R)
            keep = leaf_J[s] <= split_J
            is_leaf[s] = keep
            J = np.where(keep, leaf_J[s], split_J) + lam * SPLIT_FLAG_BITS
            R = np.where(keep, leaf_R[s], split_R) + SPLIT_FLAG_BITS
        return R, is_leaf, mode_idx

    def select(self, bits_per_element: float) -> QTAllocation:
        budget = bits_per_element * self.W.size
        d_max = max(c.D.max() for c in self.cands.values())
        unit = max(d_max, 1e-30) / (2 * self.sizes[-1] ** 2)
        lo_l, hi_l = np.log(unit * 1e-16), np.log(unit * 1e6)
        best = self._solve(np.exp(hi_l))
        if best[0].sum() > budget:
            raise ValueError(f"Budget {bits_per_element} b/elem below the minimum {best[0].sum() / self.W.size:.3f}")
        for _ in range(60):
            mid = 0.5 * (lo_l + hi_l)
            trial = self._solve(np.exp(mid))
            if trial[0].sum() <= budget:
                best, hi_l = trial, mid
            else:
                lo_l = mid
        R, is_leaf, mode_idx = best

        # a node is a final leaf iff it chose "leaf" and no ancestor did
        active = np.ones_like(is_leaf[self.sizes[0]], dtype=bool)
        leaf, modes, scales = {}, {}, {}
        for i, s in enumerate(self.sizes):
            leaf[s] = active & is_leaf[s]
            if i + 1 < len(self.sizes):
                active = _up4(active & ~is_leaf[s])
            c = self.cands[s]
            grid_modes = np.array(c.modes, dtype=np.uint8)[mode_idx[s]]
            grid_scales = np.take_along_axis(c.S, mode_idx[s][None], 0)[0]
            modes[s] = np.where(leaf[s], grid_modes, 0).astype(np.uint8)
            scales[s] = np.where(leaf[s], grid_scales, 0).astype(np.float32)
        return QTAllocation(self.sizes, leaf, modes, scales, None, int(R.sum()), weights=self.W)


def qt_allocate(W: np.ndarray, bits_per_element: float, importance: Optional[np.ndarray] = None,
                sizes: Sequence[int] = (32, 16, 8), modes: Sequence[int] = DEFAULT_MODES) -> QTAllocation:
    return QuadtreeRD(W, importance, sizes, modes).select(bits_per_element)
