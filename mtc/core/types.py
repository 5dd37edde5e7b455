"""mtc.core.types (mtc/core/types.py:9-28): precision modes of a quantized block or leaf."""

from tensorpack_amd.core.types import PrecisionMode

__all__ = ["PrecisionMode"]
