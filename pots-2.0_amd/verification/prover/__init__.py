"""A synthetic prover: a step's transcript and operands built directly in HBM."""
