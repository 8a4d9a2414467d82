"""Quantisation utilities."""
