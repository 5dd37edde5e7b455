"""mtc.core.precision (mtc/core/precision.py): the per-block precision rules of the uniform
constructors `MTCMatrix.from_numpy` / `from_numpy_joint`."""

from tensorpack_amd.core.precision import quantize_and_dequantize_block, select_independent_precision

__all__ = ["quantize_and_dequantize_block", "select_independent_precision"]
