"""CPU oracle of the BitLinear path -- test infrastructure only (see oracle.py)."""
