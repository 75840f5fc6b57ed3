"""CPU oracle for the W8A8 linear and fused DiT-norm path (test infrastructure only)."""
