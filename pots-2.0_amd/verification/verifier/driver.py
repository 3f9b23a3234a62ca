"""The verifier over one run: checks 0 and 1 at its start, the per-step checks, checks 8 and 9
at its end (reference: verification/verifier/driver.py:86-376).

The constructor takes the reference's public inputs (``C``, ``h_D`` with ``|D|``, ``k``, the
step count ``T``, the bands, the schedule seed, and the agreed ``W_0`` as tensors or leaf
hashes) and refuses what the reference refuses: both or neither ``W_0`` form, an ``h_D``
that is not a digest, ``k`` outside 1..255, no bands outside calibration, provisional bands
without ``allow_provisional``, and κ classes or τ_W tensors that name nothing in ``C``.

- :meth:`Verifier.start_run` hashes the agreed ``W_0`` on the GPU (check 0's anchor) and runs
  check 1 over the agreed ``D``: its record count and its root ``h_D``. The schedule ``π`` is
  adopted for every step when the caller passes ``schedule``; the reference's default schedule
  (a BLAKE3 shuffle of ``D`` by ``seed``, ``setup/data.py:325``) and check 4, the only check
  that reads ``π``, are not part of this build.
- :meth:`Verifier.verify_step` runs :data:`~.checks.DEFAULT_ORDER` (``7 → 2 → 6a → 5 → 6b →
  2.root``; check 7 reports as check 0 on the first step, against ``W_0``; 6b is skipped when
  check 5 measured the prover's own operands), stops at the first
  rejection, keeps each step's statistics and per-slot wall clock, and on acceptance keeps the
  step's ``W_{t+1}`` leaf hashes for the next step's check 7. With ``overlap`` (the default)
  a step is first tried on the overlapped path (:mod:`.overlap`: one read, the GPU work of
  checks 2 and 5 in flight together, judged in the same order), which only accepts; anything
  else runs the slots one at a time, which find and word the rejection.
- :meth:`Verifier.freeze` ends a calibration run by judging the recorded numbers of every
  calibrated step in check order: 6a, then 5, then 6b.
- :meth:`Verifier.end_run` compares the kept hashes with the agreed final weights (check 8,
  which a run shorter than ``T`` also fails) and returns check 9's :class:`RunVerdict`.

Check 5's operands come from ``C.replay``. A computation that serves the prover's own captured
operands instead (``DeclaredComputation.use_operands``) makes check 5 a consistency check of
what the prover sent, not a replay of the committed leaves; the verifier takes such a
computation only with ``trust_prover_operands=True`` and marks every step's statistics with it.
"""

from __future__ import annotations

import contextlib
import gc
import time
from collections.abc import Callable, Iterator, Mapping, Sequence
from contextlib import AbstractContextManager
from dataclasses import dataclass
from typing import Any

import torch

from verification.commitment.leaves import leaf_hashes_of
from verification.commitment.merkle import DIGEST_SIZE, merkle_root
from verification.computation.interface import DeclaredComputation
from verification.transcript.store import TranscriptStore
from verification.verifier.bands import Bands, product_class
from verification.verifier.checks import CHECKS, DEFAULT_ORDER, ROOT_SLOT
from verification.verifier.overlap import NOT_DECIDED, OverlapCache, decide
from verification.verifier.context import (Rejection, Section, StepContext, StepStats,
                                           no_section)
from verification.verifier.plans import PlanCache

__all__ = ["RUN_START", "RunVerdict", "Verifier"]

RUN_START = 0  # the step a rejection at run start is reported at
RECORD_NOT_RUN = "not run"


@dataclass(frozen=True)
class RunVerdict:
    """Check 9: the run is accepted iff checks 0, 1, every step's checks and 8 held;
    ``band_source`` names the bands that judged it."""

    accepted: bool
    rejection: Rejection | None
    steps_verified: int
    band_source: str | None


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


def _check_bands(bands: Bands, c: DeclaredComputation) -> None:
    """A κ class or τ_W tensor the bands name must exist in ``C``: a misspelt key would
    otherwise judge with the default band."""
    classes = {product_class(c, spec) for spec in c.products}
    extra = sorted(set(bands.kappa_classes) - classes)
    if extra:
        raise ValueError(f"bands name κ classes that match no product of C: {extra}")
    extra = sorted(set(bands.tau_w_tensors) - set(c.weight_names))
    if extra:
        raise ValueError(f"bands name τ_W tensors that match no weight of C: {extra}")


def _prover_supplied(c: DeclaredComputation) -> bool:
    return bool(getattr(getattr(c, "_operands", None), "prover_supplied", False))


class Verifier:
    """The verifier of one run; it is never given a prover object."""

    def __init__(self, computation: DeclaredComputation, *, h_D: bytes, n_records: int,
                 k: int, n_steps: int, bands: Bands | None, seed: int,
                 w0: Mapping[str, torch.Tensor] | None = None,
                 w0_hashes: Sequence[bytes] | None = None,
                 schedule: Callable[[int], Sequence[int]] | None = None,
                 calibrate: bool = False, allow_provisional: bool = False,
                 section: Section | None = None, kappa_guard: bool = True,
                 trust_prover_operands: bool = False, overlap: bool = True) -> None:
        if (w0 is None) == (w0_hashes is None):
            raise ValueError("give exactly one of w0 and w0_hashes")
        if not (isinstance(h_D, bytes) and len(h_D) == DIGEST_SIZE):
            raise ValueError("h_D must be a 32-byte digest")
        if not 1 <= k <= 255:
            raise ValueError(f"k must be in 1..255, got {k}")
        if not (isinstance(n_steps, int) and n_steps >= 1):
            raise ValueError(f"n_steps (T) must be a positive int, got {n_steps!r}")
        if bands is None and not calibrate:
            raise ValueError("bands are required outside calibration mode")
        if calibrate and not kappa_guard:
            raise ValueError("calibration fits κ_max, so it needs the κ guard on")
        if _prover_supplied(computation) and not trust_prover_operands:
            raise ValueError("the computation serves the prover's captured operands to check "
                             "5; pass trust_prover_operands=True to verify against them")
        self.c, self.h_D, self.n_records, self.k = computation, h_D, int(n_records), int(k)
        self.n_steps, self.seed = n_steps, int(seed)
        self.allow_provisional, self.calibrate = allow_provisional, calibrate
        self.kappa_guard, self.section = kappa_guard, section
        self.trust_prover_operands = trust_prover_operands
        self.overlap = overlap
        # steps accepted on the overlapped path, and steps it left to the slots
        self.overlapped: list[int] = []
        self.serial: list[int] = []
        self.bands: Bands | None = None
        if bands is not None:
            self._adopt(bands)
        self._schedule = schedule
        self._w0, self._w0_hashes = w0, None if w0_hashes is None else tuple(w0_hashes)
        self._chain: tuple[bytes, ...] | None = None  # W_{t+1} hashes kept between steps
        self._last_step = 0
        self.calibrated_steps: list[int] = []
        self.rejection: Rejection | None = None
        self.timings: dict[int, dict[str, float]] = {}
        self.run_timings: dict[str, float] = {}
        self.stats: dict[int, StepStats] = {}
        self.record_pass: dict[int, str] = {}
        # the leaf and Freivalds plans of the last step, run again while the layout repeats
        self.plans = PlanCache()

    def _adopt(self, bands: Bands) -> None:
        if bands.source == "provisional" and not self.allow_provisional:
            raise ValueError("provisional bands judge only with allow_provisional=True; a "
                             "cheat run uses the calibrated band file")
        _check_bands(bands, self.c)
        self.bands = bands

    def _timed(self, name: str) -> AbstractContextManager[Any]:
        return no_section(name) if self.section is None else self.section(name)

    @property
    def band_source(self) -> str | None:
        return None if self.calibrate or self.bands is None else self.bands.source

    # ---- run start: checks 0 and 1 ------------------------------------------------------

    def weight_hashes(self, weights: Mapping[str, torch.Tensor]) -> tuple[bytes, ...]:
        """The leaf hashes of agreed weights in ``C``'s order (tag 0x02, so they compare with
        ``W_t`` and ``W_{t+1}`` leaves alike)."""
        if set(weights) != set(self.c.weight_names):
            raise ValueError("weights differ from the declared weight names")
        return tuple(leaf_hashes_of(self.c, ((self.c.w_t_index(name), weights[name].detach())
                                             for name in self.c.weight_names)))

    def _digests(self, hashes: Sequence[bytes]) -> tuple[bytes, ...]:
        out = tuple(hashes)
        if len(out) != self.c.n_w or any(not (isinstance(h, bytes) and len(h) == DIGEST_SIZE)
                                         for h in out):
            raise ValueError(f"expected {self.c.n_w} digests of {DIGEST_SIZE} bytes")
        return out

    def start_run(self, dataset: Sequence[Any]) -> Rejection | None:
        """Check 0's anchor (the agreed ``W_0``'s hashes) and check 1 over the agreed ``D``."""
        if self._chain is not None:
            raise RuntimeError("start_run was already called")
        t0 = time.perf_counter()
        with self._timed("run:0"):
            anchor = self.weight_hashes(self._w0) if self._w0 is not None \
                else self._digests(self._w0_hashes or ())
        self.run_timings["0"] = time.perf_counter() - t0
        t0 = time.perf_counter()
        with self._timed("run:1"):
            rej = self._check_1(dataset)
        self.run_timings["1"] = time.perf_counter() - t0
        if rej is not None:
            self.rejection = rej
            return rej
        self._chain = anchor
        return None

    def _check_1(self, dataset: Sequence[Any]) -> Rejection | None:
        if len(dataset) != self.n_records:
            return Rejection(RUN_START, "1", f"D has {len(dataset)} records, the manifest "
                                             f"declares {self.n_records}")
        h = merkle_root(leaf_hashes_of(self.c, ((0, r) for r in dataset)))
        if h != self.h_D:
            return Rejection(RUN_START, "1", f"h_D over the agreed D is {h.hex()[:16]}…, "
                                             f"published {self.h_D.hex()[:16]}…")
        if self._schedule is None:
            return None
        for t in range(1, self.n_steps + 1):
            try:
                idx = list(self._schedule(t))
            except ValueError as e:
                return Rejection(RUN_START, "1", f"π({t}) is undefined: {e}")
            if len(idx) != self.c.n_s or len(set(idx)) != len(idx) or \
                    not all(0 <= i < self.n_records for i in idx):
                return Rejection(RUN_START, "1", f"π({t}) = {idx} is not {self.c.n_s} "
                                                 f"distinct indices into D")
        return None

    # ---- per step ---------------------------------------------------------------------

    def verify_step(self, t: int, store: TranscriptStore) -> Rejection | None:
        """Run the default order on step ``t`` (1-based, consecutive); ``None`` accepts."""
        if self._chain is None:
            raise RuntimeError("call start_run before verify_step")
        if self.rejection is not None:
            raise RuntimeError(f"the run is already rejected: {self.rejection}")
        if t != self._last_step + 1:
            raise RuntimeError(f"expected step {self._last_step + 1}, got {t}")
        if t > self.n_steps:
            raise RuntimeError(f"step {t} is past the declared T = {self.n_steps}")
        bands = self.bands if self.bands is not None else Bands.provisional()
        indices = tuple(self._schedule(t)) if self._schedule else ()

        def context() -> StepContext:
            return StepContext.for_computation(
                self.c, step=t, indices=indices, h_D=self.h_D, n_records=self.n_records,
                prev_w_hashes=self._chain, chain_check_id="0" if t == 1 else "7", k=self.k,
                judge=not self.calibrate, section=self.section, kappa_guard=self.kappa_guard,
                trust_prover_operands=self.trust_prover_operands, plans=self.plans)

        timings = self.timings[t] = {}
        with _collector_paused():
            decided = NOT_DECIDED
            if self.overlap:
                ctx = context()
                self.stats[t] = ctx.stats
                if self.plans.overlap is None:
                    self.plans.overlap = OverlapCache()
                with self._timed("overlap"):
                    decided = decide(self.c, store, ctx, bands, self.plans.overlap, timings)
            if decided is NOT_DECIDED:
                timings.clear()
                ctx = context()
                self.stats[t] = ctx.stats
                for slot in DEFAULT_ORDER:
                    with self._timed(slot):
                        t0 = time.perf_counter()
                        rej = CHECKS[slot](store, self.c, ctx, bands)
                        timings[slot] = time.perf_counter() - t0
                    if rej is not None:
                        self.rejection = rej
                        self.record_pass[t] = RECORD_NOT_RUN
                        self.serial.append(t)
                        return rej
                self.serial.append(t)
            else:
                self.overlapped.append(t)
        hashes = ctx.state.leaf_hashes
        assert hashes is not None
        lo = self.c.w_next_index(self.c.weight_names[0])
        self._chain = tuple(hashes[lo:lo + self.c.n_w])
        self._last_step = t
        if self.calibrate:
            self.calibrated_steps.append(t)
        return None

    # ---- calibration ----------------------------------------------------------------------

    def freeze(self, bands: Bands) -> Rejection | None:
        """End calibration with ``bands``: the calibrated steps' recorded numbers are judged
        in check order, then every later step is judged live. A live rejection stands, except
        the root comparison's, which runs after the band checks of its step: those are judged
        first."""
        if not self.calibrate:
            raise RuntimeError("freeze is only for a calibration run")
        self._adopt(bands)
        self.calibrate = False
        live = self.rejection
        if live is not None:
            if ROOT_SLOT in self.timings.get(live.step, {}):
                rej = self._rejudge(live.step, self.stats[live.step], bands)
                if rej is not None:
                    self.rejection = rej
                    return rej
            return live
        for t in self.calibrated_steps:
            rej = self._rejudge(t, self.stats[t], bands)
            if rej is not None:
                self.rejection = rej
                return rej
        return None

    @staticmethod
    def _rejudge(t: int, stats: StepStats, bands: Bands) -> Rejection | None:
        """One calibrated step's recorded numbers against ``bands``, in the slots' order:
        6a's ``ρ_max`` per linear weight, check 5's ``κ`` and normalized residuals per
        product, then 6b's ``ρ_max`` per glue weight (reference driver.py:321-341)."""
        rej = Verifier._rejudge_updates(t, stats, bands, "6a")
        if rej is None:
            rej = Verifier._rejudge_products(t, stats, bands)
        if rej is None:
            rej = Verifier._rejudge_updates(t, stats, bands, "6b")
        return rej

    @staticmethod
    def _rejudge_updates(t: int, stats: StepStats, bands: Bands,
                         check_id: str) -> Rejection | None:
        for s in stats.tensors:
            if s.check_id != check_id:
                continue
            tau_w = bands.tau_w_for(s.weight)
            if not s.rho_max <= tau_w:
                return Rejection(t, check_id, f"{s.weight}: ρ_max = {s.rho_max:.3g} > "
                                              f"τ_W = {tau_w:g}")
        return None

    @staticmethod
    def _rejudge_products(t: int, stats: StepStats, bands: Bands) -> Rejection | None:
        for p in stats.products:
            kmax = bands.kappa_for(p.cls)
            if not p.kappa <= kmax:
                return Rejection(t, "5", f"P_{p.m} ({p.name}): cancellation factor κ = "
                                         f"{p.kappa:.3g} > κ_max = {kmax:g} [{p.cls}]")
            for j, x in enumerate(p.normalized, start=1):
                if not x <= bands.tau:
                    return Rejection(t, "5", f"P_{p.m} ({p.name}), challenge j={j}: normalized "
                                             f"residual {x:.3g} > τ = {bands.tau:g}")
        return None

    # ---- run end: checks 8 and 9 --------------------------------------------------------

    def close(self) -> None:
        """Free the plans kept between steps (their device memory); a later step builds them
        again."""
        self.plans.close()

    def end_run(self, final: Mapping[str, torch.Tensor] | Sequence[bytes]) -> RunVerdict:
        """Check 8 against the agreed final weights (tensors or leaf hashes), then check 9.
        The plans kept between steps are freed."""
        self.plans.close()
        rejected_at_start = self._chain is None and self.rejection is not None
        if self.calibrate and not rejected_at_start:
            raise RuntimeError("calibration is unfrozen: call freeze(bands) before end_run")
        if self.rejection is None:
            t0 = time.perf_counter()
            with self._timed("run:8"):
                rej = self._check_8(final)
            self.run_timings["8"] = time.perf_counter() - t0
            if rej is not None:
                self.rejection = rej
        return RunVerdict(self.rejection is None, self.rejection, self._last_step,
                          self.band_source)

    def _check_8(self, final: Mapping[str, torch.Tensor] | Sequence[bytes]) -> Rejection | None:
        if self._chain is None:
            raise RuntimeError("call start_run before end_run")
        step = self._last_step
        if step != self.n_steps:
            return Rejection(step, "8", f"{step} steps verified, the run declares "
                                        f"T = {self.n_steps}")
        want = self.weight_hashes(final) if isinstance(final, Mapping) else self._digests(final)
        for name, got, w in zip(self.c.weight_names, self._chain, want):
            if got != w:
                return Rejection(step, "8", f"final W_T[{name}] differs from the agreed weights")
        return None
