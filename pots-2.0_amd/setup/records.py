"""Token records and their canonical bytes (reference: setup/records.py:20-100).

A record leaf is ``0x01 ‖ 0x10 ‖ ℓ (4 bytes, big-endian) ‖ ids ‖ targets ‖ mask``, the three
arrays int32 little-endian in C order. The same bytes are the record's leaf in the step
root ``h`` and in the dataset root ``h_D``.
"""

from __future__ import annotations

import struct
import sys
from dataclasses import dataclass

import torch

if sys.byteorder != "little":
    raise ImportError("canonical payloads are little-endian; big-endian hosts are unsupported")

TAG_RECORD = 0x01
INT32_CODE = 0x10

_U32_MAX = 2**32 - 1


class RecordError(ValueError):
    """A record breaks the token-record format, or bytes are not a canonical record."""


def _int32_vector(name: str, t: object) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise RecordError(f"{name} must be a torch.Tensor")
    if t.dtype != torch.int32 or t.dim() != 1:
        raise RecordError(f"{name} must be a 1-D int32 tensor, got {t.dtype} with {t.dim()} dims")
    return t


@dataclass(frozen=True, eq=False)
class Record:
    """Input ids, next-token targets and the loss mask of one sequence."""

    ids: torch.Tensor
    targets: torch.Tensor
    mask: torch.Tensor

    def __post_init__(self) -> None:
        n = _int32_vector("ids", self.ids).numel()
        for name in ("targets", "mask"):
            if _int32_vector(name, getattr(self, name)).numel() != n:
                raise RecordError("ids, targets and mask must have one common length")
        if not 1 <= n <= _U32_MAX:
            raise RecordError(f"record length {n} out of range")
        if not bool(((self.mask == 0) | (self.mask == 1)).all()):
            raise RecordError("mask entries must be 0 or 1")

    def __len__(self) -> int:
        return self.ids.numel()

    def __eq__(self, other: object) -> bool:
        if not isinstance(other, Record):
            return NotImplemented
        return all(torch.equal(getattr(self, f), getattr(other, f))
                   for f in ("ids", "targets", "mask"))

    __hash__ = None  # type: ignore[assignment]


def _raw(t: torch.Tensor) -> bytes:
    if not t.is_contiguous():
        raise RecordError("tensor must be contiguous")
    return t.detach().cpu().numpy().tobytes()


def encode_record(rec: Record) -> bytes:
    """The record's leaf bytes."""
    return (struct.pack(">BBI", TAG_RECORD, INT32_CODE, len(rec))
            + _raw(rec.ids) + _raw(rec.targets) + _raw(rec.mask))
