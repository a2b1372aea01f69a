"""CPU oracle for the MLX affine group-quantized linear (test infrastructure only)."""
