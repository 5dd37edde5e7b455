"""mtc.core.precision (mtc/core/precision.py): the per-block precision rules of the uniform
constructors `MTCMatrix.from_numpy` / `from_numpy_joint`, under the reference's names and
signatures (negotiate_joint_precision takes two blocks and returns (pA, pB, scale_a, scale_b))."""

from tensorpack_amd.core.precision import (compute_frobenius_error, compute_relative_error,
                                           negotiate_joint_precision_blocks as negotiate_joint_precision,
                                           quantize_and_dequantize_block, select_independent_precision)

__all__ = ["quantize_and_dequantize_block", "compute_frobenius_error", "compute_relative_error",
           "select_independent_precision", "negotiate_joint_precision"]
