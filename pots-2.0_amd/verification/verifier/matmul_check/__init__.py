"""Check 5's challenge vectors, Freivalds rows and sizing formulas."""
