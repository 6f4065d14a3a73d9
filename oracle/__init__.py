"""CPU oracle of the speculative-decode MoE hot path (test infrastructure only)."""
