"""CPU oracle of the quantized-linear hot path (test infrastructure only)."""
