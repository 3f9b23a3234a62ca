"""Protocol constants of the hot path (reference: verification/parameters.py:21-30)."""

from __future__ import annotations

import torch

LAMBDA: int = 25
LOG2_G: int = 52

UNIT_ROUNDOFF: dict[torch.dtype, float] = {
    torch.float32: 2.0**-24,
    torch.bfloat16: 2.0**-8,
    torch.float16: 2.0**-11,
}

K_DEFAULT = 9
