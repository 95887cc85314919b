"""CPU oracle of the quantized MoE hot path (test infrastructure only)."""
