"""CPU oracle of the quantized-weight matmul path (test infrastructure only)."""
