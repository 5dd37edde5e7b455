"""`mtc.kernels`: the quantized matmul (`gemm`) and accuracy metrics (`reference`)."""
