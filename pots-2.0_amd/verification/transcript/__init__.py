"""Transcript errors and the in-memory store the verifier reads (reference: verification/transcript/)."""
