"""mtc.kernels.gemm (mtc/kernels/gemm.py): `MTCMatrix` and `mtc_gemm`, computed on MI355X.

`mtc_gemm(A, B)` keeps the reference form (two MTCMatrix, returns np.ndarray fp32) and adds
a dense X (numpy or torch) times a quadtree or uniform-block MTCMatrix.
"""

from tensorpack_amd.kernels.gemm import MTCMatrix, arena_decode, arena_encode, mtc_gemm, mtc_gemm_group

__all__ = ["MTCMatrix", "mtc_gemm", "mtc_gemm_group", "arena_encode", "arena_decode"]
