"""The verifier's hot path: check 5's Freivalds measurement and verdicts, check 2's hashing."""
