"""CPU oracle of the quantized-linear path (test infrastructure only; see oracle.py)."""
