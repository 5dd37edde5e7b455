"""Drop-in import paths of the reference package (Sharexi/TensorPack `mtc`), served by
tensorpack_amd: `from mtc.kernels.gemm import MTCMatrix, mtc_gemm` and the allocator
modules `mtc.core.quadtree`, `mtc.core.permutation` and `mtc.core.allocation` resolve to
this build, whose GEMM runs on the MI355X kernels of libmtc_hip.so.

Only the quantized-matmul path is served (mtc/__init__.py exports of the reference that
belong to other subsystems, MicroTensor / PointerTensor / OpCode, are not provided).
"""

from .core.arena import MemoryArena
from .core.types import PrecisionMode

__all__ = ["PrecisionMode", "MemoryArena"]
