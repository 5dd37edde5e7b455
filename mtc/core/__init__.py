"""`mtc.core` modules of the quantized-matmul path (allocators, arena, precision modes)."""
