"""Rate-distortion (RD) block precision allocation, offline on the CPU.

Restates the allocator of mtc/core/allocation.py so that its decisions are
bit-identical to the reference's:

- code ranges / mode lattice / clipping grids: allocation.py:44-75
- block views and the quantizer (division, ties-to-even, clip): :78-94
- per-block scale search (C++ in csrc/rd_search.cpp): :97-160
- candidate tables: :182-235
- uniform-block Lagrangian selection + greedy fill: :238-326
- pair allocation and rebuild: :329-369

Distortion model: D_b(p) = sum_{rows r of block b} h_r * ||W_r - W_hat_r||^2
with h normalised to mean 1; rate R(p) = p * Bs^2 payload bits plus a fixed
per-block metadata cost (bf16 scale + mode byte = 24 bits, fp32 scale = 40).
"""

from dataclasses import dataclass
from typing import Dict, Optional, Sequence, Tuple

import numpy as np

from .. import _native

CODE_MODES = (2, 3, 4, 5, 6, 8, 16)

# mode -> (lo, hi) signed code range of a `mode`-bit two's complement code
QRANGE: Dict[int, Tuple[int, int]] = {m: (-(1 << (m - 1)), (1 << (m - 1)) - 1) for m in CODE_MODES}

META_BITS_PER_BLOCK = 32 + 8          # fp32 scale + mode byte
SCALE_FORMAT_META_BITS = {"fp32": 32 + 8, "bf16": 16 + 8}
DEFAULT_MODES = (0,) + CODE_MODES

# Clipping-ratio grids (fraction of the block abs-max mapped to the largest code
# magnitude): every grid steps by 0.025 up to 1.0.
_ALPHA_START = {2: 0.20, 3: 0.30, 4: 0.40, 5: 0.50, 6: 0.60, 8: 0.80}
_ALPHAS = {m: np.linspace(a0, 1.0, int(round((1.0 - a0) / 0.025)) + 1) for m, a0 in _ALPHA_START.items()}
_ALPHAS[16] = np.array([1.0])


def to_blocks(W: np.ndarray, Bs: int) -> np.ndarray:
    """(K, N) -> (K/Bs, N/Bs, Bs, Bs) view; [i, j] is W[i*Bs:(i+1)*Bs, j*Bs:(j+1)*Bs]."""
    K, N = W.shape
    return W.reshape(K // Bs, Bs, N // Bs, Bs).swapaxes(1, 2)


def from_blocks(Bl: np.ndarray) -> np.ndarray:
    a, b, Bs, _ = Bl.shape
    return Bl.swapaxes(1, 2).reshape(a * Bs, b * Bs)


def quantize_blocks(blocks: np.ndarray, mode: int, scales: np.ndarray) -> np.ndarray:
    """Float32 integer codes round_half_even(block / scale) clipped to the mode's range.

    A zero scale divides by one instead (its codes then multiply a zero scale).
    """
    lo, hi = QRANGE[mode]
    s = scales[..., None, None]
    divisor = np.where(s == 0, np.float32(1.0), s)
    return np.clip(np.round(blocks / divisor), lo, hi)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to 8 significant bits, ties to even (allocation.py:97-103)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    _native.rd_lib().mtc_round_sig8(_native.ptr(x, _native.c_f32p), _native.ptr(out, _native.c_f32p), x.size)
    return out


def _search_mode(blocks: np.ndarray, h_rows: np.ndarray, mode: int, round_bf16_scales: bool = False,
                 n_threads: int = 0) -> Tuple[np.ndarray, np.ndarray]:
    """Best (distortion, scale) per block for one mode, searching clip ratio x sign."""
    lo, hi = QRANGE[mode]
    qmag = float(max(-lo, hi))
    nbk, nbn, Bs, _ = blocks.shape
    nb = nbk * nbn
    flat = np.ascontiguousarray(blocks, dtype=np.float32).reshape(nb, Bs, Bs)
    hr = np.ascontiguousarray(h_rows, dtype=np.float64).reshape(nb, Bs)
    amax = np.abs(flat).max(axis=(1, 2)).astype(np.float32)
    amax = np.where(amax < 1e-30, np.float32(1.0), amax).astype(np.float32)
    signs = np.array([1.0] if mode == 16 else [1.0, -1.0], dtype=np.float32)
    alphas = _ALPHAS[mode].astype(np.float32)
    best_d = np.empty(nb, dtype=np.float64)
    best_s = np.empty(nb, dtype=np.float32)
    F, D = _native.c_f32p, _native.c_f64p
    rc = _native.rd_lib().mtc_rd_search(
        _native.ptr(flat, F), _native.ptr(hr, D), _native.ptr(amax, F), nb, Bs,
        float(lo), float(hi), qmag, _native.ptr(alphas, F), alphas.size,
        _native.ptr(signs, F), signs.size, int(bool(round_bf16_scales)), int(n_threads),
        _native.ptr(best_d, D), _native.ptr(best_s, F))
    if rc != 0:
        raise ValueError(f"scale search failed (code {rc}) for block size {Bs}")
    return best_d.reshape(nbk, nbn), best_s.reshape(nbk, nbn)


@dataclass
class RDAllocation:
    """Uniform-block allocation of one matrix; grids are indexed [row_block, col_block]."""
    modes: np.ndarray
    scales: np.ndarray
    dequant: np.ndarray
    block_size: int
    payload_bits: int
    meta_bits: int

    @property
    def bits_per_element(self) -> float:
        return (self.payload_bits + self.meta_bits) / self.dequant.size

    def mode_histogram(self) -> Dict[int, float]:
        n = self.modes.size
        return {int(m): float((self.modes == m).sum()) / n for m in DEFAULT_MODES}


@dataclass
class RDCandidates:
    """Budget-independent per-block, per-mode (distortion, scale) tables."""
    blocks: np.ndarray       # (nbk, nbn, Bs, Bs)
    D: np.ndarray            # (n_modes, nbk, nbn) float64
    S: np.ndarray            # (n_modes, nbk, nbn) float32
    R: np.ndarray            # (n_modes,) payload bits per block
    modes: Tuple[int, ...]
    block_size: int
    shape: Tuple[int, int]
    meta_bits_per_block: int = META_BITS_PER_BLOCK


def normalized_importance(importance: Optional[np.ndarray], K: int) -> np.ndarray:
    h = np.ones(K, dtype=np.float64) if importance is None else np.asarray(importance, dtype=np.float64)
    assert h.shape == (K,), f"importance must have shape ({K},), got {h.shape}"
    return h / max(h.mean(), 1e-30)


def rd_candidates(W: np.ndarray, importance: Optional[np.ndarray] = None, block_size: int = 16,
                  modes: Sequence[int] = DEFAULT_MODES, scale_format: str = "fp32",
                  n_threads: int = 0) -> RDCandidates:
    """Run the per-block, per-mode scale search for one block size."""
    assert scale_format in SCALE_FORMAT_META_BITS, scale_format
    W = np.asarray(W, dtype=np.float32)
    K, N = W.shape
    Bs = int(block_size)
    assert K % Bs == 0 and N % Bs == 0, f"shape {W.shape} not divisible by block size {Bs}"
    h = normalized_importance(importance, K)
    blocks = to_blocks(W, Bs)
    nbk, nbn = blocks.shape[:2]
    h_rows = np.broadcast_to(h.reshape(nbk, 1, Bs), (nbk, nbn, Bs))
    modes = tuple(sorted(int(m) for m in modes))
    D = np.empty((len(modes), nbk, nbn), dtype=np.float64)
    S = np.zeros((len(modes), nbk, nbn), dtype=np.float32)
    for i, m in enumerate(modes):
        if m == 0:
            # energy of the dropped block, same contraction as allocation.py:231
            D[i] = np.einsum("abrc,abr->ab", blocks.astype(np.float64) ** 2, h_rows)
        else:
            D[i], S[i] = _search_mode(blocks, h_rows, m, scale_format == "bf16", n_threads)
    R = np.array([m * Bs * Bs for m in modes], dtype=np.float64)
    return RDCandidates(blocks, D, S, R, modes, Bs, (K, N), SCALE_FORMAT_META_BITS[scale_format])


def rd_select(c: RDCandidates, bits_per_element: float) -> RDAllocation:
    """Lagrangian mode choice (64-step bisection on log lambda) + greedy fill."""
    blocks, D, S, R, modes, Bs = c.blocks, c.D, c.S, c.R, c.modes, c.block_size
    nbk, nbn = blocks.shape[:2]
    nblk = nbk * nbn
    meta_bits = c.meta_bits_per_block * nblk
    payload_budget = bits_per_element * (c.shape[0] * c.shape[1]) - meta_bits
    if payload_budget < R.min() * nblk:
        floor = (R.min() * nblk + meta_bits) / (c.shape[0] * c.shape[1])
        raise ValueError(f"Budget {bits_per_element} b/elem is below the minimum {floor:.3f} for this mode set.")
    Df = D.reshape(len(modes), -1)
    cols = np.arange(nblk)

    def pick(lam):
        return np.argmin(Df + lam * R[:, None], axis=0)

    unit = max(Df.max(), 1e-30) / R[R > 0].min()
    lo_l, hi_l = np.log(unit * 1e-16), np.log(unit * 1e4)
    best = pick(np.exp(hi_l))
    for _ in range(64):
        mid = 0.5 * (lo_l + hi_l)
        trial = pick(np.exp(mid))
        if R[trial].sum() <= payload_budget:
            best, hi_l = trial, mid
        else:
            lo_l = mid

    # spend what is left on single-block upgrades, best distortion drop per bit first
    left = payload_budget - R[best].sum()
    while left > 0:
        cur_r, cur_d = R[best], Df[best, cols]
        gain = np.full(nblk, -np.inf)
        nxt = best.copy()
        for j in range(len(modes)):
            dr = R[j] - cur_r
            ok = (dr > 0) & (dr <= left)
            g = np.where(ok, (cur_d - Df[j]) / np.where(dr > 0, dr, 1.0), -np.inf)
            better = g > gain
            gain, nxt = np.where(better, g, gain), np.where(better, j, nxt)
        b = int(np.argmax(gain))
        if not np.isfinite(gain[b]) or gain[b] <= 0:
            break
        left -= R[nxt[b]] - R[best[b]]
        best[b] = nxt[b]

    mode_grid = np.array(modes, dtype=np.uint8)[best].reshape(nbk, nbn)
    scale_grid = S.reshape(len(modes), -1)[best, cols].reshape(nbk, nbn)
    deq = np.zeros_like(blocks)
    for m in modes:
        if m == 0:
            continue
        sel = mode_grid == m
        if sel.any():
            q = quantize_blocks(blocks[sel][None], m, scale_grid[sel][None])[0]
            deq[sel] = q * scale_grid[sel][:, None, None]
    scale_grid = np.where(mode_grid == 0, 0.0, scale_grid).astype(np.float32)
    return RDAllocation(modes=mode_grid, scales=scale_grid, dequant=from_blocks(deq).astype(np.float32),
                        block_size=Bs, payload_bits=int(R[best].sum()), meta_bits=meta_bits)


def rd_allocate(W: np.ndarray, bits_per_element: float, importance: Optional[np.ndarray] = None,
                block_size: int = 16, modes: Sequence[int] = DEFAULT_MODES,
                scale_format: str = "fp32") -> RDAllocation:
    """Uniform-block allocation of W (K x N, reduction along rows) at a total budget."""
    return rd_select(rd_candidates(W, importance, block_size, modes, scale_format), bits_per_element)


def rd_allocate_pair(A: np.ndarray, B: np.ndarray, bits_per_element: float, block_size: int = 16,
                     modes: Sequence[int] = DEFAULT_MODES,
                     use_importance: bool = True) -> Tuple[RDAllocation, RDAllocation]:
    """Joint allocation for C = A @ B: each operand weighted by the other's energy along k."""
    A = np.asarray(A, dtype=np.float32)
    B = np.asarray(B, dtype=np.float32)
    h_b = (A.astype(np.float64) ** 2).sum(axis=0) if use_importance else None
    h_a = (B.astype(np.float64) ** 2).sum(axis=1) if use_importance else None
    alloc_b = rd_allocate(B, bits_per_element, h_b, block_size, modes)
    at = rd_allocate(A.T, bits_per_element, h_a, block_size, modes)
    alloc_a = RDAllocation(modes=at.modes.T.copy(), scales=at.scales.T.copy(), dequant=at.dequant.T.copy(),
                           block_size=block_size, payload_bits=at.payload_bits, meta_bits=at.meta_bits)
    return alloc_a, alloc_b


def rd_dequant(W: np.ndarray, modes: np.ndarray, scales: np.ndarray, block_size: int = 16) -> np.ndarray:
    """Rebuild the dequantized matrix from W and a stored uniform allocation."""
    blocks = to_blocks(np.asarray(W, dtype=np.float32), block_size)
    deq = np.zeros_like(blocks)
    for m in np.unique(modes):
        if m == 0:
            continue
        sel = modes == m
        q = quantize_blocks(blocks[sel][None], int(m), scales[sel][None])[0]
        deq[sel] = q * scales[sel][:, None, None]
    return from_blocks(deq).astype(np.float32)
