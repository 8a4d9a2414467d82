"""Weight packing for the ternary matmul."""
