"""CPU oracle of the recognition-head hot path (test infrastructure only)."""
