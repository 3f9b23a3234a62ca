"""Challenge vectors ``r(m, j)`` for check 5 (reference:
verification/verifier/matmul_check/challenges.py).

Vector ``j`` of product ``m`` is the keyed BLAKE3 XOF, key = the claimed root ``h``, of the
label ``0x10 ‖ m (4 bytes BE) ‖ j (1 byte)``, read as little-endian uint32 words ``w`` with
entries ``(2(w >> 8) + 1 − 2^24) / 2^24``, exact in fp32. The XOF runs on the GPU
(``libpots_mi355x``); results are GPU tensors.
"""

from __future__ import annotations

import math
import struct
from collections.abc import Sequence

import numpy as np
import torch

from verification.commitment import native

TAG_LABEL = 0x10

SIGMA_R: float = 1.0 / math.sqrt(3.0)  # std of one challenge entry, Uniform(−1, 1)

_GRID = 1 << 24


def encode_label(m: int, j: int) -> bytes:
    """Challenge label ``0x10 ‖ m(4 BE) ‖ j(1)``; ``m`` and ``j`` are 1-based."""
    if not 1 <= m < 1 << 32:
        raise ValueError(f"label m={m} out of range")
    if not 1 <= j <= 255:
        raise ValueError(f"label j={j} out of range")
    return struct.pack(">BIB", TAG_LABEL, m, j)


def _validate(h: bytes, m: int, width: int) -> None:
    if not isinstance(h, (bytes, bytearray)) or len(h) != 32:
        raise ValueError("h must be 32 bytes")
    if not 1 <= m < 1 << 32:
        raise ValueError(f"m must be in [1, 2^32), got {m}")
    if width < 1:
        raise ValueError(f"width must be >= 1, got {width}")


def _validate_j(j: int) -> None:
    if not 1 <= j <= 255:
        raise ValueError(f"j must be in [1, 255], got {j}")


def _entries(words: np.ndarray) -> np.ndarray:
    """The entry map on uint32 words, ``(2(w >> 8) + 1 − 2^24) / 2^24`` as float32 (exact):
    the definition the GPU kernel implements, for callers holding raw XOF words."""
    a = (np.asarray(words, dtype=np.uint32) >> np.uint32(8)).view(np.int32)
    a = a * np.int32(2) + np.int32(1 - _GRID)
    out = a.astype(np.float32)
    out *= np.float32(1.0 / _GRID)
    return out


def challenge_vector(h: bytes, m: int, j: int, width: int) -> torch.Tensor:
    """``r(m, j)``, float32 ``[width]``: column ``j − 1`` of :func:`challenge_matrix`."""
    _validate(h, m, width)
    _validate_j(j)
    return native.get().challenge_matrices(bytes(h), [m], j, width)[0, :, j - 1].contiguous()


def challenge_matrix(h: bytes, m: int, k: int, width: int) -> torch.Tensor:
    """The ``k`` vectors of product ``m`` as columns, float32 ``[width, k]``."""
    _validate(h, m, width)
    if not 1 <= k <= 255:
        raise ValueError(f"k must be in [1, 255], got {k}")
    return challenge_matrices(h, [m], k, width)[0]


def challenge_matrices(h: bytes, ms: Sequence[int], k: int, width: int) -> torch.Tensor:
    """``challenge_matrix(h, m, k, width)`` for each ``m``, as ``[len(ms), width, k]``."""
    if not 1 <= k <= 255:
        raise ValueError(f"k must be in [1, 255], got {k}")
    for m in ms:
        _validate(h, m, width)
    return native.get().challenge_matrices(bytes(h), list(ms), k, width)
