"""The per-step verifier for the hot path's checks (reference: verification/verifier/driver.py
:223-271, ``Verifier.verify_step``).

``verify_step(t, store)`` runs :data:`checks.DEFAULT_ORDER` (``2 → 6a → 5 → 2.root``) on step
``t`` with one :class:`StepContext`, stops at the first rejection and keeps it, and keeps the
step's statistics and per-slot timings as the reference does (``stats[t]``, ``timings[t]``).
The run-level state of the reference's verifier (the data schedule, the weight-hash chain,
checks 0, 1, 4, 6b, 7 and 8, the record pass after a rejection) is not part of this build.
"""

from __future__ import annotations

import contextlib
import gc
import time
from collections.abc import Iterator
from typing import Any

from verification.computation.interface import DeclaredComputation
from verification.transcript.store import TranscriptStore
from verification.verifier.bands import Bands
from verification.verifier.checks import CHECKS, DEFAULT_ORDER
from verification.verifier.context import Rejection, StepContext, StepStats

__all__ = ["Verifier"]


@contextlib.contextmanager
def _collector_paused() -> Iterator[None]:
    """Python's cyclic collector off for one step: the step allocates tens of thousands of
    small objects (a row per product, a stat per leaf), and each collection it would trigger
    scans the whole heap of transcript objects. Reference counting still frees everything;
    cycles wait for the next collection."""
    was = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if was:
            gc.enable()


class Verifier:
    """Checks 2, 6a, 5 and 2.root of consecutive steps of one run under one computation."""

    def __init__(self, c: DeclaredComputation, *, k: int, bands: Bands | None = None,
                 calibrate: bool = False, kappa_guard: bool = True,
                 section: Any = None) -> None:
        if not 1 <= k <= 255:
            raise ValueError(f"k must be in [1, 255], got {k}")
        self.c, self.k, self.bands = c, k, bands
        self.calibrate, self.kappa_guard, self.section = calibrate, kappa_guard, section
        self.rejection: Rejection | None = None
        self.stats: dict[int, StepStats] = {}
        self.timings: dict[int, dict[str, float]] = {}
        self._last_step = 0

    def verify_step(self, t: int, store: TranscriptStore) -> Rejection | None:
        """Run the default order on step ``t`` (1-based, consecutive); ``None`` accepts."""
        if self.rejection is not None:
            raise RuntimeError(f"the run is already rejected: {self.rejection}")
        if t != self._last_step + 1:
            raise RuntimeError(f"expected step {self._last_step + 1}, got {t}")
        bands = self.bands if self.bands is not None else Bands.provisional()
        ctx = StepContext.for_computation(
            self.c, step=t, indices=(), h_D=b"", n_records=0, prev_w_hashes=(),
            chain_check_id="7", k=self.k, judge=not self.calibrate, section=self.section,
            kappa_guard=self.kappa_guard)
        timings = self.timings[t] = {}
        self.stats[t] = ctx.stats
        with _collector_paused():
            for slot in DEFAULT_ORDER:
                t0 = time.perf_counter()
                rej = CHECKS[slot](store, self.c, ctx, bands)
                timings[slot] = time.perf_counter() - t0
                if rej is not None:
                    self.rejection = rej
                    return rej
        self._last_step = t
        return None
