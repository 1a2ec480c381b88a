"""CPU oracle for the quantized matmul path (test infrastructure only; see oracle.py)."""
