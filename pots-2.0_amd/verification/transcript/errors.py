"""Errors raised by prover data that does not fit the declared transcript format
(reference: verification/transcript/errors.py). The verifier maps each to a rejection at
the check that read the leaf."""

from __future__ import annotations

__all__ = ["TranscriptFormatError", "LeafShapeError", "LeafDtypeError", "StoreMutationError",
           "LeafReadError"]


class TranscriptFormatError(ValueError):
    """Prover data that doesn't fit the declared transcript format."""


class LeafShapeError(TranscriptFormatError):
    """A leaf's shape differs from the one its slot declares."""


class LeafDtypeError(TranscriptFormatError):
    """A leaf's dtype differs from the one its slot declares."""


class StoreMutationError(TranscriptFormatError):
    """A stored leaf was changed in place after handoff."""


class LeafReadError(TranscriptFormatError):
    """A stored leaf or the store's metadata can't be read back."""
