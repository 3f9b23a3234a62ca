"""Deterministic leaf payloads for the golden digests: the same bytes on every machine.

Values are standard normal from numpy's PCG64 at the given seed, rounded to the dtype by
torch (round to nearest even), or int32 from the same generator.
"""

from __future__ import annotations

import math

import numpy as np
import torch

# The reference's edge shapes around its 64 KiB block (tests/verification/commitment/
# test_native.py:56-57), plus chunk-boundary sizes of the BLAKE3 tree.
SHAPES = [(0,), (1,), (3,), (7, 5), (253,), (256,), (16383,), (16384,), (16385,),
          (3, 5461, 3), (262143,), (262144,), (262145,), (5, 1 << 18)]
DTYPES = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16,
          "int32": torch.int32}


def payload(shape: tuple[int, ...], dtype: torch.dtype, seed: int) -> torch.Tensor:
    n = math.prod(shape)
    rng = np.random.default_rng(seed)
    if dtype == torch.int32:
        return torch.from_numpy(rng.integers(-2**31, 2**31, size=n, dtype=np.int64)
                                .astype(np.int32)).reshape(shape)
    return torch.from_numpy(rng.standard_normal(n, dtype=np.float32)).to(dtype).reshape(shape)
