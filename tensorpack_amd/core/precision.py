"""Per-block precision rules of the reference's legacy uniform constructors.

`MTCMatrix.from_numpy` (mtc/kernels/gemm.py:255-328) picks each block's mode either
from a fixed `precision_mode` or by the independent epsilon rule, and
`MTCMatrix.from_numpy_joint` (gemm.py:330-430) by negotiating the modes of every
interacting (A, B) block pair. The rules below restate mtc/core/precision.py and the
quantizer of MicroTensor.from_array (mtc/core/microtensor.py:63-160) with the same
float32/float64 operations, so the arenas they produce hold the reference's bytes.
"""

from typing import Dict, Optional, Tuple

import numpy as np

from .types import PrecisionMode

# symmetric code magnitude per mode: scale = max|block| / QMAG (microtensor.py:83-92)
QMAG = {2: 1.0, 4: 7.0, 8: 127.0, 16: 32767.0}
# code range per mode written by MicroTensor.from_array
CLIP = {2: (-2, 1), 4: (-8, 7), 8: (-128, 127), 16: (-32768, 32767)}
NEGOTIATED_MODES = (2, 4, 8, 16)


def quantize_and_dequantize_block(block: np.ndarray, mode: int) -> Tuple[np.ndarray, float]:
    """(reconstruction, scale) of one block at `mode` (precision.py:11-41): codes are
    round(block / scale) clipped to the mode's range, scale = max|block| / QMAG[mode]
    (a Python float); an all-but-zero block (max < 1e-8) reconstructs to zeros with scale 1."""
    arr = np.asarray(block, dtype=np.float32)
    max_abs = float(np.max(np.abs(arr)))
    if max_abs < 1e-8:
        return np.zeros_like(arr), 1.0
    if mode not in QMAG:
        raise ValueError(f"Unknown precision: {mode}")
    scale = max_abs / QMAG[mode]
    lo, hi = CLIP[mode]
    q = np.clip(np.round(arr / scale), lo, hi).astype(np.int16 if mode == 16 else np.int8)
    return q.astype(np.float32) * scale, scale


def _frobenius_error(orig: np.ndarray, recon: np.ndarray) -> float:
    return float(np.linalg.norm(orig.astype(np.float32) - recon.astype(np.float32)))


def _relative_error(orig: np.ndarray, recon: np.ndarray) -> float:
    n = float(np.linalg.norm(orig))
    return 0.0 if n < 1e-8 else _frobenius_error(orig, recon) / n


def select_independent_precision(block: np.ndarray, epsilon: float = 0.05) -> Tuple[PrecisionMode, float]:
    """The lowest of P2, P4, P8 whose relative reconstruction error is <= epsilon, with its
    scale; otherwise P16 with scale 1.0 (precision.py:58-74)."""
    for mode in (2, 4, 8):
        recon, scale = quantize_and_dequantize_block(block, mode)
        if _relative_error(block, recon) <= epsilon:
            return PrecisionMode(mode), scale
    return PrecisionMode.P16, 1.0


class _BlockErrors:
    """Frobenius norm, per-mode reconstruction error and scale of one block (computed once;
    the negotiation below asks for them once per interacting pair)."""

    def __init__(self, block: np.ndarray):
        self.norm = float(np.linalg.norm(block))
        self.err: Dict[int, float] = {}
        self.scale: Dict[int, float] = {}
        for m in NEGOTIATED_MODES:
            rec, sc = quantize_and_dequantize_block(block, m)
            self.err[m] = _frobenius_error(block, rec)
            self.scale[m] = sc


# candidate (pA, pB) pairs ordered by pA + pB, then max(pA, pB) (stable: ties keep pA-major order)
_PAIRS = sorted(((a, b) for a in NEGOTIATED_MODES for b in NEGOTIATED_MODES), key=lambda p: (p[0] + p[1], max(p)))


def negotiate_joint_precision(ea: _BlockErrors, eb: _BlockErrors, target_epsilon: float = 0.05,
                              reduction_tiles: int = 1) -> Tuple[int, int]:
    """Modes (pA, pB) of an interacting block pair (precision.py:77-140): the cheapest pair,
    in the order above, whose product-error bound ea*|B| + |A|*eb + ea*eb is within
    target_epsilon / sqrt(reduction_tiles) * |A||B|; (P2, P2) when |A||B| < 1e-7; else (P16, P16)."""
    norm_ab = ea.norm * eb.norm
    if norm_ab < 1e-7:
        return 2, 2
    allowed = (target_epsilon / np.sqrt(max(1, reduction_tiles))) * norm_ab
    for pa, pb in _PAIRS:
        a, b = ea.err[pa], eb.err[pb]
        if a * eb.norm + ea.norm * b + a * b <= allowed:
            return pa, pb
    return 16, 16


def compute_frobenius_error(orig: np.ndarray, recon: np.ndarray) -> float:
    """||orig - recon||_F in float32 (precision.py:44-47)."""
    return _frobenius_error(orig, recon)


def compute_relative_error(orig: np.ndarray, recon: np.ndarray) -> float:
    """||orig - recon||_F / ||orig||_F, 0 for a block of norm < 1e-8 (precision.py:50-55)."""
    return _relative_error(orig, recon)


def negotiate_joint_precision_blocks(block_a: np.ndarray, block_b: np.ndarray, target_epsilon: float = 0.05,
                                     reduction_tiles: int = 1) -> Tuple[PrecisionMode, PrecisionMode, float, float]:
    """The reference's form of the negotiation (precision.py:77-140): two blocks in, (pA, pB,
    scale_a, scale_b) out, with scales 1.0 for a pair whose |A||B| < 1e-7."""
    ea, eb = _BlockErrors(block_a), _BlockErrors(block_b)
    if ea.norm * eb.norm < 1e-7:
        return PrecisionMode.P2, PrecisionMode.P2, 1.0, 1.0
    pa, pb = negotiate_joint_precision(ea, eb, target_epsilon, reduction_tiles)
    return PrecisionMode(pa), PrecisionMode(pb), ea.scale[pa], eb.scale[pb]


def block_scale(block: np.ndarray, mode: int, scale: Optional[float] = None) -> float:
    """The scale MicroTensor.from_array stores for `block` (microtensor.py:80-92): the given
    one, else max|block| / QMAG[mode], or 1.0 for a block whose max is <= 1e-7."""
    if scale is not None:
        return scale
    max_abs = float(np.max(np.abs(np.asarray(block, dtype=np.float32))))
    return max_abs / QMAG[mode] if max_abs > 1e-7 else 1.0


def block_codes(block: np.ndarray, mode: int, scale: float) -> np.ndarray:
    """Signed codes MicroTensor.from_array writes (microtensor.py:94-151): the float32 block
    times float32(1 / scale) (1 when the scale is 0), rounded half to even and clipped."""
    if mode not in CLIP:
        raise ValueError(f"Unsupported precision: {mode}")
    arr = np.asarray(block, dtype=np.float32)
    inv = 1.0 / scale if scale != 0.0 else 1.0
    lo, hi = CLIP[mode]
    return np.clip(np.round(arr * inv), lo, hi).astype(np.int32)
