"""BitLinear layers."""
