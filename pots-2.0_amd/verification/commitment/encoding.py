"""Canonical leaf bytes (reference: verification/commitment/encoding.py:19-126).

A tensor leaf is ``tag(1) ‖ dtype(1) ‖ ndim(1) ‖ dim_0 … dim_{ndim−1} (4 bytes each,
big-endian)`` followed by the tensor's raw little-endian C-order payload. Tags: 0x02 weight,
0x03 product, 0x04 MLP record. Float leaves holding NaN or Inf are rejected; ``-0.0`` passes.

Unlike the reference, a payload may live in HBM: ``tensor_payload_span`` returns a device
address for a CUDA tensor, and the GPU hashing kernels read it in place.
"""

from __future__ import annotations

import struct
import sys

import torch

if sys.byteorder != "little":
    raise ImportError("canonical payloads are little-endian; big-endian hosts are unsupported")

TAG_WEIGHT = 0x02
TAG_PRODUCT = 0x03
TAG_MLP_RECORD = 0x04

TENSOR_TAGS = frozenset({TAG_WEIGHT, TAG_PRODUCT, TAG_MLP_RECORD})

DTYPE_CODES: dict[torch.dtype, int] = {
    torch.float32: 0x01,
    torch.bfloat16: 0x02,
    torch.float16: 0x03,
    torch.int32: 0x10,
}
CODE_DTYPES: dict[int, torch.dtype] = {v: k for k, v in DTYPE_CODES.items()}
FLOAT_DTYPES = frozenset({torch.float32, torch.bfloat16, torch.float16})

_U32_MAX = 2**32 - 1


class NonFiniteError(ValueError):
    """A float tensor bound for a commitment holds NaN or Inf."""


class EncodingError(ValueError):
    """An object cannot be canonically encoded, or bytes are not a canonical encoding."""


def tensor_leaf_header(tag: int, t: torch.Tensor) -> bytes:
    """``tag ‖ dtype ‖ ndim ‖ dims (BE u32)``."""
    if tag not in TENSOR_TAGS:
        raise EncodingError(f"tag {tag:#x} is not a tensor-leaf tag")
    if t.dtype not in DTYPE_CODES:
        raise EncodingError(f"dtype {t.dtype} has no canonical code")
    shape = tuple(t.shape)
    if len(shape) > 255:
        raise EncodingError("ndim exceeds 255")
    if any(d > _U32_MAX for d in shape):
        raise EncodingError("dimension exceeds uint32")
    return struct.pack(f">BBB{len(shape)}I", tag, DTYPE_CODES[t.dtype], len(shape), *shape)


def _all_finite(t: torch.Tensor) -> bool:
    """``torch.isfinite(t).all()``: both extremes are finite exactly when every entry is."""
    if t.numel() == 0:
        return True
    lo, hi = torch.aminmax(t)
    return bool(lo.isfinite() & hi.isfinite())


def _check_payload(t: torch.Tensor) -> None:
    """A coded dtype and a contiguous layout; the tensor may be on the CPU or the GPU."""
    if t.dtype not in DTYPE_CODES:
        raise EncodingError(f"dtype {t.dtype} has no canonical code")
    if t.device.type not in ("cpu", "cuda"):
        raise EncodingError(f"tensor must be on the CPU or a GPU, got {t.device}")
    if not t.is_contiguous():
        raise EncodingError("tensor must be contiguous")


def _payload_view(t: torch.Tensor) -> memoryview:
    t = t.detach()
    if t.device.type != "cpu":
        t = t.cpu()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return memoryview(t.reshape(-1).numpy()).cast("B")


def tensor_leaf_payload(t: torch.Tensor) -> memoryview:
    """Byte view of the payload (a host copy for a GPU tensor). NaN/Inf raise
    ``NonFiniteError``."""
    _check_payload(t)
    if t.dtype in FLOAT_DTYPES and not _all_finite(t.detach()):
        raise NonFiniteError("float tensor contains NaN or Inf")
    return _payload_view(t)


def tensor_leaf_payload_unchecked(t: torch.Tensor) -> memoryview:
    """``tensor_leaf_payload`` without the finiteness check."""
    _check_payload(t)
    return _payload_view(t)


def tensor_payload_span(t: torch.Tensor) -> tuple[int, int]:
    """``(address, byte length)`` of the payload, in host or device memory. The caller keeps
    ``t`` alive and unmodified until hashing is done."""
    _check_payload(t)
    return t.data_ptr(), t.nbytes


def encode_tensor_leaf(tag: int, t: torch.Tensor) -> bytes:
    """Full leaf bytes as one host copy, for small tensors and tests."""
    return tensor_leaf_header(tag, t) + bytes(tensor_leaf_payload(t))
