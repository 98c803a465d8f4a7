"""CPU oracle for the Q4_K/Q6_K x Q8_K path (test infrastructure only)."""
