"""mtc.kernels.reference (mtc/kernels/reference.py:10-54): host accuracy metrics."""

from tensorpack_amd.kernels.reference import (fp32_gemm_numpy, max_absolute_error, relative_frobenius_error,
                                              signal_to_noise_ratio_db)

__all__ = ["fp32_gemm_numpy", "relative_frobenius_error", "max_absolute_error", "signal_to_noise_ratio_db"]
