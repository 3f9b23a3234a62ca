"""Plans kept from one verified step to the next while the transcript's layout repeats.

Building a leaf plan or a Freivalds plan is host work that grows with the leaf and product
counts (C4: about 7 ms and 10-15 ms in the library, and the Python tables before that). Steps
of one run have the same shapes, and a transcript written into the same device buffers step
after step (a loader's arena, the caching allocator's blocks for the same sequence of
allocations) has the same addresses too. A plan depends on nothing else, so the verifier keeps
the plans of its last step and runs them again when the next step's layout is byte for byte
the same: every header, payload address, length and finiteness kind for a leaf plan; every
operand address, leading dimension, shape, dtype and label for a Freivalds plan.

A cached plan keeps no tensor between steps: it would keep the previous step's transcript
alive. A run is enqueued only after the key matched, that is with every address it reads
holding this step's tensor, and the caller keeps those tensors until the run's results are
read. The tensors the Freivalds table itself makes for each step (a biased product's fp32
bias, a row-major copy of an operand in another layout, such as a replay's transposed view)
are keyed by position instead of address, and their values are copied into the ones the cached
plan points at.

The cache holds device memory (at C4 about 2 GB for the check-2 leaf plan's workspace and
1.3 GB for the Freivalds plan) until :meth:`PlanCache.close` or the process ends.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass, field
from typing import Any

import numpy as np
import torch

from verification.commitment import native

__all__ = ["PlanCache"]


@dataclass
class _FvEntry:
    key: bytes
    plan: native.FvPlan
    made: dict[tuple[int, str], torch.Tensor] = field(default_factory=dict)


class PlanCache:
    """The last leaf plan of each hashing site (keyed by the caller's ``site`` name: check 7
    and check 2 hash different leaves) and the last Freivalds plan."""

    def __init__(self) -> None:
        self._leaf: dict[str, tuple[bytes, native.LeafPlan]] = {}
        self._fv: _FvEntry | None = None
        self.hits = 0
        self.builds = 0
        # the overlapped path's plans (verification.verifier.overlap.OverlapCache)
        self.overlap: Any = None

    def leaf_plan(self, site: str, hdr_buf: bytes, hdr_off: np.ndarray, hdr_len: np.ndarray,
                  hdr_idx: np.ndarray, payload_ptr: np.ndarray, payload_len: np.ndarray,
                  kind: np.ndarray, device: torch.device) -> native.LeafPlan:
        """A leaf plan over ``pots_hash_leaves``'s arguments, every payload in device memory:
        the cached one if the arguments are the same, else a new one (the old one closed)."""
        arrays = [np.ascontiguousarray(hdr_off, dtype=np.uint64),
                  np.ascontiguousarray(hdr_len, dtype=np.uint32),
                  np.ascontiguousarray(hdr_idx, dtype=np.uint32),
                  np.ascontiguousarray(payload_ptr, dtype=np.uint64),
                  np.ascontiguousarray(payload_len, dtype=np.uint64),
                  np.ascontiguousarray(kind, dtype=np.uint8)]
        sizes = np.array([len(hdr_buf), *(a.nbytes for a in arrays), device.index or 0],
                         dtype=np.uint64)
        key = b"".join([sizes.tobytes(), hdr_buf, *(a.tobytes() for a in arrays)])
        got = self._leaf.get(site)
        if got is not None and got[0] == key:
            self.hits += 1
            return got[1]
        if got is not None:
            got[1].close()
            del self._leaf[site]
        plan = native.LeafPlan.from_arrays(native.get(), hdr_buf, *arrays, device)
        self._leaf[site] = (key, plan)
        self.builds += 1
        return plan

    def fv_plan(self, products: Sequence[native.FvProduct], k: int,
                guard: bool) -> native.FvPlan:
        """A Freivalds plan over ``products``: the cached one if the product table is the same
        (with the addresses of the tensors the table makes, a bias or a row-major copy, left
        out), those tensors' values refreshed; else a new one. The plan holds this step's
        operands until :meth:`release`."""
        arr, keep, made = native.fv_table(products, k)
        keyed = arr.copy()
        for i, f in made:
            keyed[f][i] = 1
        key = b"".join([np.array([k, int(bool(guard))], dtype=np.uint64).tobytes(),
                        keyed.tobytes()])
        e = self._fv
        if e is not None and e.key == key and e.made.keys() == made.keys():
            for at, t in made.items():
                e.made[at].copy_(t)
            e.plan._keep = keep
            self.hits += 1
            return e.plan
        if e is not None:
            e.plan.close()
            self._fv = None
        plan = native.FvPlan(native.get(), products, k, guard, table=(arr, keep, made))
        self._fv = _FvEntry(key, plan, made)
        self.builds += 1
        return plan

    @staticmethod
    def release(plan: native.FvPlan | native.LeafPlan) -> None:
        """Drop the plan's references to this step's tensors once its results are read."""
        plan._keep = []

    def close(self) -> None:
        if self.overlap is not None:
            self.overlap.close()
        for _, plan in self._leaf.values():
            plan.close()
        self._leaf.clear()
        if self._fv is not None:
            self._fv.plan.close()
            self._fv = None
