"""Host-side accuracy metrics of the reference API (mtc/kernels/reference.py:10-54).

These measure results; they compute nothing on the GEMM path itself.
"""

import numpy as np


def fp32_gemm_numpy(A: np.ndarray, B: np.ndarray) -> np.ndarray:
    """Plain fp32 BLAS product."""
    return np.matmul(np.asarray(A, dtype=np.float32), np.asarray(B, dtype=np.float32))


def relative_frobenius_error(y_true: np.ndarray, y_pred: np.ndarray) -> float:
    """||y_true - y_pred||_F / ||y_true||_F in float64; the absolute norm when ||y_true|| < 1e-12."""
    t = np.asarray(y_true, dtype=np.float64)
    diff = np.linalg.norm(t - np.asarray(y_pred, dtype=np.float64))
    ref = np.linalg.norm(t)
    return float(diff) if ref < 1e-12 else float(diff / ref)


def max_absolute_error(y_true: np.ndarray, y_pred: np.ndarray) -> float:
    return float(np.max(np.abs(np.asarray(y_true, np.float64) - np.asarray(y_pred, np.float64))))


def signal_to_noise_ratio_db(y_true: np.ndarray, y_pred: np.ndarray) -> float:
    t = np.asarray(y_true, np.float64)
    noise = np.mean((t - np.asarray(y_pred, np.float64)) ** 2)
    signal = np.mean(t ** 2)
    if noise < 1e-15:
        return 120.0
    if signal < 1e-15:
        return 0.0
    return float(10.0 * np.log10(signal / noise))
