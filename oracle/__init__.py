"""CPU oracle of the reference Gefen path (test infrastructure only)."""
