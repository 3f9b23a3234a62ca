"""One step's check 2 and check 5 on a transcript resident in HBM, in one pass of the GPU.

Reference: verification/verifier/checks.py:204-272 (check 2's read-hash-validate and its root
comparison) and :576-956 (check 5: challenges keyed on the claimed root, Freivalds
measurement of every product in canonical order, judging). The checks' order of effects is
kept: a non-finite leaf is check 2's malformed rejection; otherwise the first product that
fails its tests is check 5's rejection; otherwise a root that differs from the claim rejects
as check 2 at the end (F15a: check 5 keys on the claimed root, so it need not wait for the
recomputed one).

What runs where. Check 2's hashing (leaf digests, then the Merkle tree) and check 5's
measuring (challenges, the three Freivalds passes, rows) depend only on the leaves and the
claimed root, so they run on two streams at once: hashing is integer-VALU bound and uses a
fraction of HBM bandwidth, the Freivalds passes are memory bound and leave the VALUs mostly
idle. Each product's P is a leaf, so by default the leaf plan is fused with the Freivalds plan
(``pots_leaf_plan_create_fused``): the chunk kernel takes the P-pass sums of the product leaves
it streams and P is read once. The challenges then go first, the chunk kernel waits for them,
and the P stage (which adds up the chunk kernel's run records) waits for the chunk kernel. The
verdicts follow on the main stream. One host read at the end returns the root, the first
non-finite leaf and the first rejected product.
"""

from __future__ import annotations

from collections.abc import Callable, Sequence
from dataclasses import dataclass
from typing import Any

import torch

from verification.commitment import native
from verification.commitment.leaves import StepHasher
from verification.computation.interface import DeclaredComputation
from verification.parameters import UNIT_ROUNDOFF
from verification.verifier.bands import Bands, product_class

CODE_NAMES = {0: "accept", 1: "non-finite", 2: "cancellation", 3: "residual"}


@dataclass
class StepVerdict:
    """The outcome of one step's checks 2 and 5."""

    root: bytes                 # the recomputed Merkle root
    first_bad: int              # first leaf holding NaN/Inf, or n_leaves
    first_fail: int             # index (0-based, canonical order) of the first rejected product, or M
    codes: torch.Tensor         # int32 [M, 2]: (code, failing challenge j) per product
    rows: torch.Tensor          # fp64 [M, 5 + k] Freivalds rows (freivalds.ROW)
    check: str | None           # "2", "5" or None (accept)
    detail: str | None


# The A stage's grid beside the fused chunk kernel, as multiples of the CU count (0: one block
# per tile, no limit). Results do not depend on it (pots_fv_plan_set_grid); the time does.
A_GRID_CANDIDATES = (1.0, 1.5, 2.0, 0.0)


def calibrate_a_grid(plan: native.FvPlan, run: Callable[[], tuple[Any, Any]],
                     device: torch.device, reps: int = 2) -> tuple[int, dict[int, float]]:
    """The A stage's grid for this plan: each candidate of :data:`A_GRID_CANDIDATES` timed on
    the step itself (``run`` enqueues one whole step and returns its start and end CUDA
    events, recorded with timing), after one untimed run, best of ``reps``; the fastest is set
    on the plan and returned with the table of times (ms). The rule replaces a model of the
    two halves' rates: which grid lets the hashing and the A stage finish together depends on
    the shapes, the fused share of the hashing and the host's gaps, and the step measures it
    directly, once per plan."""
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    times: dict[int, float] = {}
    for f in A_GRID_CANDIDATES:
        g = int(round(f * cus))
        if g in times:
            continue
        plan.set_grid(3, g)
        events = [run() for _ in range(reps + 1)]
        torch.cuda.synchronize(device)
        times[g] = min(s.elapsed_time(e) for s, e in events[1:])
    best = min(times, key=lambda g: (times[g], g))
    plan.set_grid(3, best)
    return best, times


def enqueue_measure_and_hash(plan: native.FvPlan, hp: native.LeafPlan, fused: int,
                             key: torch.Tensor, digests: torch.Tensor, bad: torch.Tensor,
                             rows: torch.Tensor, side: torch.cuda.Stream,
                             start: torch.cuda.Event, *, timing: bool = False,
                             hash_after_b: bool = True, plain_early: bool = False
                             ) -> tuple[torch.cuda.Event, ...]:
    """Check 5's Freivalds stages on the current stream and check 2's chunk stages on
    ``side`` (after ``start``), as one step runs them: with a fused leaf plan, the challenges
    and the unfused P pass first, then the B pass and reduce, then the fused chunk kernel
    beside the A stage, and the fused products' sums once the chunk kernel is done; the rows
    last. The leaf plan's levels and the tree are the caller's (on ``side``, after this).
    Returns the events (chunks begin, chunks end, A begin, A end)."""
    main = torch.cuda.current_stream()
    c_begin = torch.cuda.Event(enable_timing=timing)
    c_end = torch.cuda.Event(enable_timing=timing)
    a_begin = torch.cuda.Event(enable_timing=timing)
    a_end = torch.cuda.Event(enable_timing=timing)
    side.wait_event(start)
    if not fused:
        with torch.cuda.stream(side):
            hp.run_stage(0, digests, bad, side)
            c_begin.record(side)
            hp.run_stage(1, digests, bad, side)
            c_end.record(side)
        for st in range(5):
            if st == 3:
                a_begin.record(main)
            plan.run_stage(st, key, rows, main)
            if st == 3:
                a_end.record(main)
    else:
        # The fused chunk kernel reads the challenges and, started after the B pass, shares
        # the CUs with a bounded A pass; the other leaves' chunks go first.
        with torch.cuda.stream(side):
            hp.run_stage(0, digests, bad, side)
            if plain_early:
                hp.run_stage(native.LeafPlan.PLAIN_CHUNKS, digests, bad, side)
        # The unfused products' P pass needs only the challenges: it goes first, so that the
        # step's end waits only for the fused products' sums.
        plan.run_stage(0, key, rows, main)
        plan.run_stage(native.FvPlan.P_PASS, key, rows, main)
        for st in range(1, 3 if hash_after_b else 1):
            plan.run_stage(st, key, rows, main)
        ready = torch.cuda.Event()
        ready.record(main)
        side.wait_event(ready)
        with torch.cuda.stream(side):
            c_begin.record(side)
            hp.run_stage(native.LeafPlan.FUSED_CHUNKS, digests, bad, side)
            c_end.record(side)
            if not plain_early:
                hp.run_stage(native.LeafPlan.PLAIN_CHUNKS, digests, bad, side)
        for st in range(3 if hash_after_b else 1, 4):
            if st == 3:
                a_begin.record(main)
            plan.run_stage(st, key, rows, main)
        a_end.record(main)
        # the fused products' sums add up the chunk kernel's run records
        main.wait_event(c_end)
        plan.run_stage(native.FvPlan.P_FUSED, key, rows, main)
    return c_begin, c_end, a_begin, a_end


class DeviceStepVerifier:
    """Plans for one step's transcript, built once: the leaf-hashing plan, the Freivalds plan
    over every product (operands served by ``operands(spec)``), and the verdict table. Call
    :meth:`run` with the claimed root."""

    def __init__(self, c: DeclaredComputation, leaves: Sequence[Any], operands: Any, *, k: int,
                 bands: Bands | None = None, guard: bool = True, fuse: bool = True,
                 a_grid: int | None = None, b_grid: int = 0, hash_after_b: bool = True,
                 plain_early: bool = False) -> None:
        self.c, self.k, self.guard = c, k, guard
        self.bands = bands or Bands.provisional()
        lib = self.lib = native.get()
        prods = []
        for spec in c.products:
            a, b = operands(spec)
            p = leaves[c.product_index(spec.m)]
            bias = None
            if spec.bias is not None:  # checks.py:439: the W_t leaf in the operand format
                bias = leaves[c.w_t_index(spec.bias)].to(c.operand_dtype).to(torch.float32)
            prods.append(native.FvProduct(a, b, p, spec.m, bias))
        self.plan = lib.fv_plan(prods, k, guard)
        # A bounded A pass (``a_grid`` blocks, 0: one per tile) leaves room on every CU for the
        # hashing kernels beside it; by default the grid is timed on the step once
        # (calibrate_a_grid).
        self.hash_after_b, self.plain_early = hash_after_b, plain_early
        # Fused: the chunk kernel takes the P-pass sums of the product leaves it hashes, so
        # each P is read from HBM once (pots_leaf_plan_create_fused).
        self.hasher = StepHasher(c, leaves, fuse=self.plan if fuse else None)
        self.fused = self.hasher.plan.fused
        self.plan.set_grid(1, b_grid)
        self.grid_times: dict[int, float] = {}
        self.specs = native.verdict_specs(
            [s.q for s in c.products], [s.a_shape[0] for s in c.products],
            [s.bias is not None for s in c.products],
            [self.bands.kappa_for(product_class(c, s)) for s in c.products])
        self.eps_in = UNIT_ROUNDOFF[c.product_dtype]
        self.eps_acc = UNIT_ROUNDOFF[torch.float32]
        dev = self.hasher.plan.device
        self.digests = torch.empty(c.n_leaves, 32, dtype=torch.uint8, device=dev)
        self.bad = torch.empty(1, dtype=torch.int32, device=dev)
        self.rows = torch.empty(c.M, 5 + k, dtype=torch.float64, device=dev)
        self.key = torch.empty(32, dtype=torch.uint8, device=dev)
        self.side = torch.cuda.Stream(device=dev)
        self.hash_bytes = self.hasher.bytes
        self.freivalds_bytes = self.plan.bytes
        if a_grid is None and self.fused:
            zero = torch.zeros(32, dtype=torch.uint8, device=dev)

            def run() -> tuple[Any, Any]:
                ev: list = []
                self.enqueue(zero, ev)
                return ev[0][0], ev[0][3]

            a_grid, self.grid_times = calibrate_a_grid(self.plan, run, dev)
        else:
            a_grid = a_grid or 0
            self.plan.set_grid(3, a_grid)
        self.a_grid = a_grid

    def close(self) -> None:
        """Free the plans' device memory (the leaf plan first: the Freivalds plan it may be
        fused with must outlive it)."""
        self.hasher.plan.close()
        self.plan.close()

    def enqueue(self, claimed: bytes | torch.Tensor, events: list | None = None):
        """Enqueue the whole step on the current stream (Freivalds, verdicts) and a side
        stream (hashing, tree); returns GPU tensors ``(nodes, codes, first_fail)``.
        ``events``, if given, receives (start, hashed, measured, judged, chunks_begin,
        chunks_end, a_begin, a_end) CUDA events: chunks_* bracket the chunk kernel on the side
        stream, a_* the A pass on the current stream."""
        main = torch.cuda.current_stream()
        if isinstance(claimed, torch.Tensor):
            self.key.copy_(claimed)
        else:
            self.key.copy_(torch.frombuffer(bytearray(claimed), dtype=torch.uint8))
        timing = events is not None
        start = torch.cuda.Event(enable_timing=timing)
        start.record(main)
        ev = enqueue_measure_and_hash(self.plan, self.hasher.plan, self.fused, self.key,
                                      self.digests, self.bad, self.rows, self.side, start,
                                      timing=timing, hash_after_b=self.hash_after_b,
                                      plain_early=self.plain_early)
        c_begin, c_end, a_begin, a_end = ev
        plan, hp, side = self.plan, self.hasher.plan, self.side
        with torch.cuda.stream(side):
            hp.run_stage(2, self.digests, self.bad, side)
            nodes = self.lib.merkle_tree_device(self.digests, side)
        hashed = torch.cuda.Event(enable_timing=events is not None)
        hashed.record(side)
        plan.run_stage(5, self.key, self.rows, main)
        measured = torch.cuda.Event(enable_timing=events is not None)
        measured.record(main)
        main.wait_event(hashed)
        codes, _, first = self.lib.verdicts(self.rows, self.specs, k=self.k, eps_in=self.eps_in,
                                            eps_acc=self.eps_acc, tau=self.bands.tau,
                                            guard=self.guard, stream=main)
        judged = torch.cuda.Event(enable_timing=events is not None)
        judged.record(main)
        # keep the side stream's tensors alive for the main stream's consumers
        nodes.record_stream(main)
        if events is not None:
            events.append((start, hashed, measured, judged, c_begin, c_end, a_begin, a_end))
        return nodes, codes, first

    def run(self, claimed: bytes) -> StepVerdict:
        """The step's verdict, after one host read."""
        nodes, codes, first = self.enqueue(claimed)
        flags = torch.cat([nodes[0].view(torch.int32), self.bad, first]).cpu()
        root = flags[:8].numpy().tobytes()
        first_bad, first_fail = int(flags[8]), int(flags[9])
        check = detail = None
        c = self.c
        if first_bad < c.n_leaves:
            check, detail = "2", f"leaf {first_bad}: float tensor contains NaN or Inf"
        elif first_fail < c.M:
            code, j = codes[first_fail].tolist()
            spec = c.products[first_fail]
            detail = f"P_{spec.m} ({spec.name}): {CODE_NAMES[code]}" + (
                f", challenge j={j}" if code == 3 else "")
            check = "5"
        elif root != bytes(claimed):
            check, detail = "2", (f"recomputed root {root.hex()[:16]}… != claimed "
                                  f"{bytes(claimed).hex()[:16]}…")
        return StepVerdict(root, first_bad, first_fail, codes, self.rows, check, detail)
