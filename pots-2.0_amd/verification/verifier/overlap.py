"""One step's checks with check 2's hashing and check 5's measuring on the GPU at once: the
accept path of :meth:`~verification.verifier.driver.Verifier.verify_step`.

Reference: verification/verifier/driver.py:223-263 runs the default order's slots one after
another (checks.py:159-197 check 7, :204-272 check 2, :454-467 check 6a, :576-658 check 5,
:960-995 check 6b). Run that way, each slot waits for its own GPU work and reads its leaves
and operands object by object. This path reads every leaf once, serves the products one
operand group at a time (``c.operand_groups``: a batched attention product's members come as
its whole operands), keeps the step's plans while the leaves and operands lie where the last
step's did (every address, shape, stride and dtype compared), and enqueues the whole step as
:class:`~verification.verifier.step.DeviceStepVerifier` does: check 5's challenges keyed on
the claimed root (F15a), the Freivalds passes on the current stream, check 2's hashing and
tree on a side stream with the product leaves' P-pass sums taken by the chunk kernel, check
6a's update pass, and one host read. The results are judged in the default order 7 → 2 → 6a →
5 → 6b → 2.root, recording the step's statistics as the slots do.

It decides acceptance only. Whenever a check would not pass, or the step is not in the form
this path takes (a record that is a tensor, a leaf off the GPU or not as its slot declares, an
error from the store or the replay), it returns :data:`NOT_DECIDED`, and the caller runs the
slots one at a time on a fresh read: they find the rejection the reference's order makes and
word it as the reference does. A step is accepted here only when every check passed on the
bytes of this one read.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from time import perf_counter
from typing import Any

import numpy as np
import torch

from verification.commitment import native
from verification.commitment.leaves import _slot_table
from verification.transcript.store import TranscriptStore
from verification.verifier.bands import Bands
from verification.verifier.checks import CHECKS, _product_table, judge_rows
from verification.verifier.context import CommittedLeaves, StepContext, TensorStat, _is_digest
from verification.verifier.step import calibrate_a_grid

__all__ = ["NOT_DECIDED", "OverlapCache", "decide"]


class _NotDecided:
    def __repr__(self) -> str:
        return "NOT_DECIDED"


NOT_DECIDED: Any = _NotDecided()

_BF16 = native._DT[torch.bfloat16]
_MADE = 1  # a made tensor's address in a layout key: keyed by position, not address


@dataclass
class _Entry:
    """The plans and buffers of one layout."""

    leaf_key: bytes
    fv_key: bytes
    made: dict[tuple[int, str], torch.Tensor]
    fv: native.FvPlan
    leaf: native.LeafPlan
    records: torch.Tensor                 # the records' bytes, refreshed every step
    record_at: list[tuple[int, int]]      # (offset, length) of each record in it
    bias: torch.Tensor | None             # the biases in the operand format, as fp32
    update: native.UpdatePlan | None
    update_key: bytes
    specs_key: bytes = b""
    specs: torch.Tensor | None = None
    buffers: dict[str, torch.Tensor] = field(default_factory=dict)
    grid_times: dict[int, float] = field(default_factory=dict)  # A-stage grid → step ms

    def close(self) -> None:
        self.leaf.close()  # before the Freivalds plan it is fused with
        self.fv.close()
        if self.update is not None:
            self.update.close()


class OverlapCache:
    """The plans of the last step decided on the overlapped path."""

    def __init__(self) -> None:
        self.entry: _Entry | None = None
        self.hits = 0
        self.builds = 0
        self.declined: str | None = None  # why the last step was left to the slots

    def close(self) -> None:
        if self.entry is not None:
            self.entry.close()
            self.entry = None


@dataclass
class _Layout:
    """Per computation: where each product's P, bias and challenges come from."""

    p_leaf: np.ndarray       # the leaf index of each product's P
    n: np.ndarray
    q: np.ndarray            # A's columns (without the bias)
    w: np.ndarray
    m: np.ndarray
    bias_names: list[str]    # the distinct biases, in order of first use
    bias_of: np.ndarray      # per product: its bias's offset (floats) in the bias buffer, or -1
    bias_floats: int
    w_t_slots: np.ndarray    # W_t leaf indices, in weight order
    slot_dtypes: list[torch.dtype]   # what each tensor leaf's slot declares
    slot_shapes: list[torch.Size]
    headers_ok: bool                 # every slot's dtype has a leaf encoding


_LAYOUTS: dict[int, tuple[Any, _Layout]] = {}


def _layout(c: Any) -> _Layout:
    got = _LAYOUTS.get(id(c))
    if got is not None and got[0] is c:
        return got[1]
    specs = c.products
    slots = _slot_table(c)
    names: list[str] = []
    at: dict[str, int] = {}
    floats = 0
    bias_of = np.full(len(specs), -1, dtype=np.int64)
    for i, s in enumerate(specs):
        if s.bias is not None:
            if s.bias not in at:
                at[s.bias] = floats
                names.append(s.bias)
                floats += s.b_shape[1]
            bias_of[i] = at[s.bias]
    lay = _Layout(
        p_leaf=np.array([c.product_index(s.m) for s in specs], dtype=np.int64),
        n=np.array([s.a_shape[0] for s in specs], dtype=np.int64),
        q=np.array([s.a_shape[1] for s in specs], dtype=np.int64),
        w=np.array([s.b_shape[1] for s in specs], dtype=np.int64),
        m=np.array([s.m for s in specs], dtype=np.int64),
        bias_names=names, bias_of=bias_of, bias_floats=floats,
        w_t_slots=np.array([c.w_t_index(nm) for nm in c.weight_names], dtype=np.int64),
        slot_dtypes=[sl.dtype for sl in slots], slot_shapes=[sl.shape for sl in slots],
        headers_ok=all(sl.header is not None for sl in slots))
    _LAYOUTS[id(c)] = (c, lay)
    return lay


def _operand(x: torch.Tensor, rows: int, cols: int) -> tuple[int, int, int, int, int] | None:
    """Where ``x`` (``[rows, cols]`` or a stack ``[g, rows, cols]``) lies: ``(first member's
    address, bytes from one member to the next, leading dimension, 1 if each member is the
    transpose of a row-major [cols, rows] else 0, dtype code)``, or ``None`` for a layout the
    plan does not read in place."""
    dt = native._DT.get(x.dtype)
    if dt is None or not x.is_cuda:
        return None
    if x.dim() == 2:
        sg, (s0, s1) = 0, x.stride()
    else:
        sg, s0, s1 = x.stride()
    es = x.element_size()
    if s1 == 1 and (s0 >= cols or rows == 1):
        return x.data_ptr(), sg * es, s0, 0, dt
    if s0 == 1 and rows > 1 and s1 >= rows:
        return x.data_ptr(), sg * es, s1, 1, dt
    return None


class _Served:
    """The product table of one step, built a group at a time: each group's operands as
    (first address, step between members, leading dimension, ...), spread over its members'
    rows at the end."""

    def __init__(self, c: Any, lay: _Layout, leaf_ptr: np.ndarray, k: int) -> None:
        self.c, self.lay, self.k = c, lay, k
        M = c.M
        self.rows = np.zeros(M, dtype=native._FV_RECORD)
        self.rows["n"] = lay.n
        self.rows["q"] = lay.q
        self.rows["w"] = lay.w
        self.rows["m"] = lay.m
        self.rows["p"] = leaf_ptr[lay.p_leaf]
        self.rows["ldp"] = lay.w
        self.rows["p_dtype"] = native._DT[c.product_dtype]
        self.keep: list[torch.Tensor] = []
        self.made: dict[tuple[int, str], torch.Tensor] = {}
        self.groups: list[tuple[int, ...]] = []
        self.a: list[tuple[int, int, int, int, int]] = []
        self.b: list[tuple[int, int, int, int, int]] = []
        self.operands_a: list[torch.Tensor] = []

    def add(self, gi: int, grp: tuple[int, ...], a: torch.Tensor, b: torch.Tensor) -> None:
        lay = self.lay
        i0 = grp[0]
        n, q, w = int(lay.n[i0]), int(lay.q[i0]), int(lay.w[i0])
        la = _operand(a, n, q)
        if la is None or (la[3] and not self._may_twin(la, n, q)):
            a = self.copy(gi, "a", a)
            la = _operand(a, n, q)
        lb = _operand(b, q, w)
        if lb is None or lb[3]:
            b = self.copy(gi, "b", b)
            lb = _operand(b, q, w)
        if la is None or lb is None:
            raise ValueError(f"group {gi}: operands the plan cannot read")
        self.groups.append(grp)
        self.a.append(la)
        self.b.append(lb)
        self.operands_a.append(a)
        self.keep += [a, b]

    def _may_twin(self, la: tuple[int, int, int, int, int], n: int, q: int) -> bool:
        # The twin pass's terms (native._twin_mates): bf16, k ≤ 4, X = Aᵀ with rows a
        # multiple of 16 and columns of 128, 16-byte aligned rows.
        base, step, ld, _, dt = la
        return (dt == _BF16 and 1 <= self.k <= 4 and q % 16 == 0 and n % 128 == 0 and
                (2 * ld) % 16 == 0 and base % 16 == 0 and step % 16 == 0)

    def copy(self, gi: int, name: str, x: torch.Tensor) -> torch.Tensor:
        t = x.contiguous()
        self.made[(gi, name)] = t
        return t

    def finish(self) -> None:
        """Spread each group's operands over its members' rows, then give each transposed A
        its row-major mate (the same X, once); a group with a member left without one is
        copied to row-major."""
        rows = self.rows
        counts = np.array([len(g) for g in self.groups], dtype=np.int64)
        idx = np.fromiter((i for g in self.groups for i in g), dtype=np.int64,
                          count=int(counts.sum()))
        start = np.cumsum(counts) - counts
        within = (np.arange(len(idx), dtype=np.int64) - np.repeat(start, counts)) \
            .astype(np.uint64)
        for name, ops in (("a", self.a), ("b", self.b)):
            t = np.array(ops, dtype=np.uint64).reshape(-1, 5)
            ptr = np.repeat(t[:, 0], counts) + within * np.repeat(t[:, 1], counts)
            rows[name][idx] = ptr
            rows["ld" + name][idx] = np.repeat(t[:, 2], counts)
            rows[name + "_dtype"][idx] = np.repeat(t[:, 4], counts)
            if name == "a":
                rows["a_trans"][idx] = np.repeat(t[:, 3], counts)
        for gi in self._lost():
            grp = np.asarray(self.groups[gi], dtype=np.int64)
            i0 = int(grp[0])
            a = self.copy(gi, "a", self.operands_a[gi])
            la = _operand(a, int(self.lay.n[i0]), int(self.lay.q[i0]))
            if la is None:
                raise ValueError(f"group {gi}: A the plan cannot read")
            rows["a"][grp] = np.uint64(la[0]) + np.arange(len(grp), dtype=np.uint64) * \
                np.uint64(la[1])
            rows["lda"][grp] = la[2]
            rows["a_trans"][grp] = 0
            self.keep.append(a)

    def _lost(self) -> list[int]:
        """The groups with a transposed A that some member has no mate for."""
        rows = self.rows
        cand = np.flatnonzero(rows["a_trans"] == 1)
        if cand.size == 0:
            return []
        rm = np.flatnonzero((rows["a_trans"] == 0) & (rows["a_dtype"] == _BF16))
        order = np.argsort(rows["a"][rm], kind="stable")
        rm_sorted = rm[order]
        rm_ptr = rows["a"][rm_sorted]
        at = np.searchsorted(rm_ptr, rows["a"][cand])
        found = at < rm_ptr.size
        j = rm_sorted[np.minimum(at, max(rm_ptr.size - 1, 0))] if rm_ptr.size else at
        if rm_ptr.size:
            found &= rm_ptr[np.minimum(at, rm_ptr.size - 1)] == rows["a"][cand]
            found &= (rows["n"][j] == rows["q"][cand]) & (rows["q"][j] == rows["n"][cand]) \
                & (rows["lda"][j] == rows["lda"][cand])
        unique = rm_ptr.size < 2 or bool(np.all(np.diff(rm_ptr) != 0))
        if not unique or np.unique(j[found]).size != int(found.sum()):
            found = self._mates_one_by_one(cand)  # a shared X: each mate taken once, in order
        owner = np.empty(len(rows), dtype=np.int64)
        for gi, grp in enumerate(self.groups):
            owner[list(grp)] = gi
        return sorted(set(owner[cand[~found]].tolist()))

    def _mates_one_by_one(self, cand: np.ndarray) -> np.ndarray:
        rows = self.rows
        rm = np.flatnonzero((rows["a_trans"] == 0) & (rows["a_dtype"] == _BF16))
        by_ptr: dict[int, list[int]] = {}
        for j, p in zip(rm.tolist(), rows["a"][rm].tolist()):
            by_ptr.setdefault(p, []).append(j)
        taken: set[int] = set()
        found = np.zeros(cand.size, dtype=bool)
        n, q, ld, ptr = rows["n"], rows["q"], rows["lda"], rows["a"]
        for t, i in enumerate(cand.tolist()):
            for j in by_ptr.get(int(ptr[i]), ()):
                if j not in taken and n[j] == q[i] and q[j] == n[i] and ld[j] == ld[i]:
                    taken.add(j)
                    found[t] = True
                    break
        return found


def decide(c: Any, store: TranscriptStore, ctx: StepContext, bands: Bands,
           cache: OverlapCache, timings: dict[str, float]) -> Any:
    """Accept step ``ctx.step`` (``None``, with ``ctx`` filled as the slots fill it) or
    return :data:`NOT_DECIDED`; never a rejection (see the module)."""
    cache.declined = None

    def no(reason: str, wait: torch.cuda.Stream | None = None,
           alone: native.FvPlan | None = None) -> Any:
        cache.declined = reason
        return _undecided(wait, alone)

    if c.M == 0:
        return no("no products")
    t0 = perf_counter()
    # ---- one read of every leaf, in order (checks 7 and 2 judge the same objects): each
    # tensor leaf on one GPU as its slot declares, the records' bytes
    n_s = c.n_s
    lay = _layout(c)
    try:
        leaf = store.leaf
        objs = [leaf(i) for i in range(c.n_leaves)]
        leaves = CommittedLeaves.of(objs)
        claimed = store.root
        tensors = objs[n_s:]
        if not (all([isinstance(o, torch.Tensor) for o in tensors]) and
                [o.dtype for o in tensors] == lay.slot_dtypes and
                [o.shape for o in tensors] == lay.slot_shapes and
                all([o.is_cuda for o in tensors]) and
                all([o.is_contiguous() for o in tensors])):
            return no("a tensor leaf is not on the GPU as its slot declares")
        devices = {o.get_device() for o in tensors}
        if len(devices) != 1 or any(c.record_leaf(objs[i]) is not None for i in range(n_s)):
            return no("leaves on several devices, or records that are tensor leaves")
        dev_index = devices.pop()
        leaf_ptr = np.zeros(c.n_leaves, dtype=np.uint64)
        leaf_ptr[n_s:] = np.fromiter((o.data_ptr() for o in tensors), dtype=np.uint64,
                                     count=len(tensors))
        records = [c.encode_record(objs[i]) for i in range(n_s)]
    except Exception as e:
        return no(f"reading the leaves: {type(e).__name__}: {e}")
    if not _is_digest(claimed) or not lay.headers_ok:
        return no("the claimed root is not a digest, or a slot's dtype has no encoding")
    dev = torch.device("cuda", dev_index)
    ctx.state.leaves, ctx.state.claimed_root = leaves, claimed
    rec_len = np.array([len(r) for r in records], dtype=np.uint64)
    leaf_key = b"".join([rec_len.tobytes(), leaf_ptr[n_s:].tobytes(),
                         np.array([dev_index], dtype=np.uint64).tobytes()])
    t1 = perf_counter()
    timings["read"] = t1 - t0

    # ---- on the last step's leaf layout, the work that reads only leaves starts now, beside
    # the serving: check 5's challenges and the unfused products' P pass, check 6a's update
    # pass, check 2's staging
    lib = native.get()
    main = torch.cuda.current_stream(dev)
    e = cache.entry
    early = e is not None and e.leaf_key == leaf_key
    update = upd = None
    if early:
        try:
            update = _update_plan(c, e, objs, leaf_key, ctx, bands)
        except (ValueError, RuntimeError) as err:
            return no(f"check 6a's plan: {err}")
        buf = e.buffers
        key = buf["key"]
        _stage_records(e, records)
        key.copy_(torch.frombuffer(bytearray(claimed), dtype=torch.uint8))
        start = torch.cuda.Event()
        start.record(main)
        _enqueue_hashing(e, key, start)
        if update is not None:  # it reads leaves only: it runs while the products are served
            upd = update.run(buf["update"], main)

    # ---- check 5's operands, a group at a time
    wait = main if early else None
    try:
        replay = c.replay(leaves)
    except Exception as err:
        return no(f"the replay: {type(err).__name__}: {err}", wait)
    ctx.state.replay = replay
    if getattr(replay, "prover_supplied", False):
        if not ctx.trust_prover_operands:
            raise RuntimeError("check 5 was given the prover's captured operands without "
                               "trust_prover_operands")
        ctx.stats.operands_from_prover = True
    served = _Served(c, lay, leaf_ptr, ctx.k)
    specs = c.products
    try:
        for gi, grp in enumerate(c.operand_groups):
            s0 = specs[grp[0]]
            if len(grp) == 1:
                a, b = replay.operands(s0.m)
                if a.shape != s0.a_shape or b.shape != s0.b_shape:
                    return no(f"{s0.name}: served operands of other shapes", wait)
            else:
                a, b = replay.operand_group([specs[i].m for i in grp])
                g = len(grp)
                if a.shape != (g, *s0.a_shape) or b.shape != (g, *s0.b_shape):
                    return no(f"{s0.name}: a served group of other shapes", wait)
            served.add(gi, grp, a, b)
        served.finish()
    except Exception as err:
        return no(f"serving the products: {type(err).__name__}: {err}", wait)
    bias = None
    if lay.bias_names:
        bias = torch.cat([objs[c.w_t_index(nm)].reshape(-1) for nm in lay.bias_names]) \
            .to(c.operand_dtype).to(torch.float32)
    keyed = served.rows.copy()
    for (gi, name) in served.made:
        keyed[name][np.asarray(c.operand_groups[gi])] = _MADE
    keyed["bias"][lay.bias_of >= 0] = _MADE
    fv_key = b"".join([np.array([ctx.k, int(ctx.kappa_guard)], dtype=np.uint64).tobytes(),
                       keyed.tobytes()])
    t2 = perf_counter()
    timings["serve"] = t2 - t1

    # ---- check 5's passes: on the last step's plan when every operand lies where it did
    alone = None  # a plan of this step's own, when the operands moved under early hashing
    if early and e.fv_key == fv_key and e.made.keys() == served.made.keys():
        _refresh(e, served, bias)
        cache.hits += 1
        _enqueue_measuring(e, key)
    elif early:
        # The operands moved, the leaves did not (a replay rebuilt for the step allocates its
        # operands anew): the kept leaf plan hashes as planned (its fused kernel still reads
        # the kept plan's challenges, and its sums go unused), and this step is measured on a
        # Freivalds plan of its own, freed once its rows are read.
        table = served.rows.copy()
        keep = list(served.keep)
        if bias is not None:
            table["bias"] = _bias_pointers(lay, bias)
            keep.append(bias)
        try:
            alone = native.FvPlan.from_table(lib, table, keep, ctx.k, ctx.kappa_guard, dev)
        except (ValueError, RuntimeError) as err:
            return no(f"the Freivalds plan: {err}", main)
        _enqueue_chunks(e)
        alone.rows(key, buf["rows"], main)
    else:
        cache.close()
        try:
            e = _build(c, served, bias, records, objs, leaf_key, fv_key, ctx, dev)
        except (ValueError, RuntimeError) as err:  # a layout the plans refuse
            return no(f"the plans: {err}")
        cache.entry = e
        cache.builds += 1
        try:
            update = _update_plan(c, e, objs, leaf_key, ctx, bands)
        except (ValueError, RuntimeError) as err:
            return no(f"check 6a's plan: {err}")
        buf = e.buffers
        key = buf["key"]
        _stage_records(e, records)
        key.copy_(torch.frombuffer(bytearray(claimed), dtype=torch.uint8))
        if e.leaf.fused:  # the A stage's grid, timed on this step's own schedule
            _, e.grid_times = calibrate_a_grid(e.fv, lambda: _timed_run(e, key, update), dev)
        start = torch.cuda.Event()
        start.record(main)
        _enqueue_hashing(e, key, start)
        if update is not None:
            upd = update.run(buf["update"], main)
        _enqueue_measuring(e, key)

    # the verdict table: the bands' κ_max per product
    classes, qs, ns, biased = _product_table(c)
    kappa_of = {cls: bands.kappa_for(cls) for cls in set(classes)}
    kappa_max = np.array([kappa_of[cls] for cls in classes], dtype=np.float64)
    if e.specs is None or e.specs_key != kappa_max.tobytes():
        e.specs = native.verdict_specs(qs, ns, biased, kappa_max, device=dev)
        e.specs_key = kappa_max.tobytes()
    t3 = perf_counter()
    timings["plans"] = t3 - t2

    # ---- the tree, the rows, check 6a and the verdicts; one host read
    side = buf["side"]
    digests, bad, rows = buf["digests"], buf["bad"], buf["rows"]
    with torch.cuda.stream(side):
        e.leaf.run_stage(2, digests, bad, side)
        nodes = lib.merkle_tree_device(digests, side)
    hashed = torch.cuda.Event()
    hashed.record(side)
    if alone is None:
        e.fv.run_stage(5, key, rows, main)
    main.wait_event(hashed)
    nodes.record_stream(main)
    _, _, first = lib.verdicts(rows, e.specs, k=ctx.k, eps_in=ctx.eps_in, eps_acc=ctx.eps_acc,
                               tau=bands.tau, guard=ctx.kappa_guard, judge=ctx.judge,
                               stream=main)
    flags = torch.cat([nodes[0].view(torch.int32), bad.view(torch.int32),
                       first.view(torch.int32)])
    host = {name: buf["h_" + name] for name in ("flags", "digests", "rows", "update")}
    host["flags"].copy_(flags, non_blocking=True)
    host["digests"].copy_(digests, non_blocking=True)
    host["rows"].copy_(rows, non_blocking=True)
    if update is not None:
        host["update"].copy_(upd, non_blocking=True)
    main.synchronize()
    if alone is not None:
        alone.close()
    t4 = perf_counter()
    timings["gpu"] = t4 - t3

    # ---- judging, in the default order
    fl = host["flags"].numpy()
    root = fl[:8].tobytes()
    first_bad, device_first = int(fl[8]), int(fl[9])
    dig = host["digests"].numpy()
    # 7 (0 on the first step): the W_t leaves hash to the kept digests
    if len(ctx.prev_w_hashes) != c.n_w:
        raise RuntimeError(f"{len(ctx.prev_w_hashes)} chained hashes for {c.n_w} weights")
    if dig[lay.w_t_slots].tobytes() != b"".join(ctx.prev_w_hashes):
        return no(f"check {ctx.chain_check_id} would not pass")
    # 2: every leaf finite, none written in place since it was read
    if first_bad < c.n_leaves or leaves.first_changed() is not None:
        return no("check 2 would not pass")
    raw = dig.tobytes()
    ctx.state.leaf_hashes = [raw[i:i + 32] for i in range(0, 32 * c.n_leaves, 32)]
    # 6a
    if update is not None:
        res = native.UpdatePlan.decode(host["update"])
        for nm, (rho_max, first_nf, first_over) in zip(c.linear_weights, res):
            if first_nf is not None or (ctx.judge and first_over is not None):
                return no("check 6a would not pass")
            ctx.stats.tensors.append(TensorStat(nm, "6a", rho_max))
    # 5
    if judge_rows(c, host["rows"].numpy(), device_first, kappa_max, ctx, bands) is not None:
        return no("check 5 would not pass")
    # 6b (over the replay's glue; nothing to do for the prover's operands)
    if CHECKS["6b"](store, c, ctx, bands) is not None:
        return no("check 6b would not pass")
    # 2.root
    ctx.state.recomputed_root = root
    if root != claimed:
        return no("the root comparison would not pass")
    timings["judge"] = perf_counter() - t4
    return None


def _update_plan(c: Any, e: _Entry, objs: list[Any], leaf_key: bytes, ctx: StepContext,
                 bands: Bands) -> native.UpdatePlan | None:
    """Check 6a's update pass over the linear weights (leaves only), kept with the leaf
    layout and the bands; ``None`` when ``C`` declares no linear weight. Raises what the plan
    refuses."""
    names = list(c.linear_weights)
    if not names:
        return None
    taus = np.array([bands.tau_w_for(nm) for nm in names], dtype=np.float64)
    ukey = b"".join([leaf_key, taus.tobytes(),
                     np.array([c.eta, ctx.eps_w], dtype=np.float64).tobytes()])
    if e.update is None or e.update_key != ukey:
        if e.update is not None:
            e.update.close()
            e.update = None
        weights = [native.UpdateWeight(objs[c.w_t_index(nm)], objs[c.w_next_index(nm)],
                                       [objs[c.product_index(m)]
                                        for m in c.linear_weights[nm]], float(tau))
                   for nm, tau in zip(names, taus)]
        e.update = native.get().update_plan(weights, c.eta, ctx.eps_w)
        e.update._keep = []
        e.update_key = ukey
    return e.update


def _undecided(main: torch.cuda.Stream | None, alone: native.FvPlan | None = None) -> Any:
    """Leave the step to the slots once the work already enqueued for it (on both streams)
    is done."""
    if main is not None:
        torch.cuda.synchronize(main.device)
    if alone is not None:
        alone.close()
    return NOT_DECIDED


def _stage_records(e: _Entry, records: list[bytes]) -> None:
    """This step's records, each at its offset in the staged buffer (stream-ordered)."""
    if not records:
        return
    staged = np.zeros(e.records.numel(), dtype=np.uint8)
    for (o, n), r in zip(e.record_at, records):
        staged[o:o + n] = np.frombuffer(r, dtype=np.uint8)
    e.records.copy_(torch.from_numpy(staged))


def _bias_pointers(lay: _Layout, bias: torch.Tensor) -> np.ndarray:
    at = np.uint64(bias.data_ptr()) + lay.bias_of.astype(np.uint64) * np.uint64(4)
    return np.where(lay.bias_of >= 0, at, np.uint64(0))


def _refresh(e: _Entry, served: _Served, bias: torch.Tensor | None) -> None:
    """This step's values into the tensors the kept plan reads by position."""
    for at, t in served.made.items():
        e.made[at].copy_(t)
    if bias is not None:
        e.bias.copy_(bias)


def _enqueue_hashing(e: _Entry, key: torch.Tensor, start: torch.cuda.Event) -> None:
    """What needs no operand, enqueued while the products are served: check 5's challenges
    and unfused P pass on the current stream; check 2's staging on the side stream (and, for
    an unfused leaf plan, its chunk kernel). The fused chunk kernel waits for the B pass and
    the other leaves' chunks follow it (:func:`_enqueue_measuring`): started earlier, the
    chunk kernels would take every CU from the B pass and leave the A stage's tail alone."""
    main = torch.cuda.current_stream()
    buf = e.buffers
    side, digests, bad, rows = buf["side"], buf["digests"], buf["bad"], buf["rows"]
    side.wait_event(start)
    with torch.cuda.stream(side):
        e.leaf.run_stage(0, digests, bad, side)
        if not e.leaf.fused:
            e.leaf.run_stage(1, digests, bad, side)
    e.fv.run_stage(0, key, rows, main)
    e.fv.run_stage(native.FvPlan.P_PASS, key, rows, main)


def _enqueue_chunks(e: _Entry) -> torch.cuda.Event | None:
    """A fused leaf plan's chunk kernels on the side stream, after what the current stream
    has enqueued so far: the fused one, then the other leaves'. Returns the fused kernel's
    end (``None`` for an unfused plan, whose chunks :func:`_enqueue_hashing` enqueued)."""
    if not e.leaf.fused:
        return None
    main = torch.cuda.current_stream()
    buf = e.buffers
    side, digests, bad = buf["side"], buf["digests"], buf["bad"]
    ready = torch.cuda.Event()
    ready.record(main)
    side.wait_event(ready)
    c_end = torch.cuda.Event()
    with torch.cuda.stream(side):
        e.leaf.run_stage(native.LeafPlan.FUSED_CHUNKS, digests, bad, side)
        c_end.record(side)
        e.leaf.run_stage(native.LeafPlan.PLAIN_CHUNKS, digests, bad, side)
    return c_end


def _enqueue_measuring(e: _Entry, key: torch.Tensor) -> None:
    """The B pass and its reduction on the current stream; then the fused chunk kernel and
    the other leaves' chunks on the side stream beside the A stage, and the fused products'
    sums once the fused chunk kernel is done."""
    main = torch.cuda.current_stream()
    rows = e.buffers["rows"]
    e.fv.run_stage(1, key, rows, main)
    e.fv.run_stage(2, key, rows, main)
    c_end = _enqueue_chunks(e)
    e.fv.run_stage(3, key, rows, main)
    if c_end is not None:
        main.wait_event(c_end)
        e.fv.run_stage(native.FvPlan.P_FUSED, key, rows, main)


def _timed_run(e: _Entry, key: torch.Tensor, update: native.UpdatePlan | None
               ) -> tuple[torch.cuda.Event, torch.cuda.Event]:
    """One whole step in this path's order, bracketed by timing events (for the grid)."""
    main = torch.cuda.current_stream()
    buf = e.buffers
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(main)
    _enqueue_hashing(e, key, start)
    if update is not None:
        update.run(buf["update"], main)
    _enqueue_measuring(e, key)
    side = buf["side"]
    with torch.cuda.stream(side):
        e.leaf.run_stage(2, buf["digests"], buf["bad"], side)
    hashed = torch.cuda.Event()
    hashed.record(side)
    e.fv.run_stage(5, key, buf["rows"], main)
    main.wait_event(hashed)
    end.record(main)
    return start, end


def _build(c: Any, served: _Served, bias: torch.Tensor | None, records: list[bytes],
           objs: list[Any], leaf_key: bytes, fv_key: bytes, ctx: StepContext,
           dev: torch.device) -> _Entry:
    """The plans and buffers of a new layout."""
    lib = native.get()
    rows = served.rows
    keep = list(served.keep)
    lay = served.lay
    if bias is not None:
        bias = bias.clone()
        rows["bias"] = _bias_pointers(lay, bias)
        keep.append(bias)
    made = dict(served.made)
    fv = native.FvPlan.from_table(lib, rows, keep, ctx.k, ctx.kappa_guard, dev)
    # records staged in HBM, each 16-byte aligned
    at_list, off = [], 0
    for r in records:
        at_list.append((off, len(r)))
        off += (len(r) + 15) // 16 * 16
    rec_buf = torch.zeros(max(off, 16), dtype=torch.uint8, device=dev)
    slots = _slot_table(c)
    headers = [b""] * len(records) + [s.header for s in slots]
    kinds = [0] * len(records) + [s.kind for s in slots]
    uniq: dict[bytes, int] = {}
    hdr_idx = np.array([uniq.setdefault(h, len(uniq)) for h in headers], dtype=np.uint32)
    hdrs = list(uniq)
    hdr_len = np.array([len(h) for h in hdrs], dtype=np.uint32)
    hdr_off = np.zeros(len(hdrs), dtype=np.uint64)
    if len(hdrs) > 1:
        hdr_off[1:] = np.cumsum(hdr_len[:-1], dtype=np.uint64)
    ptr = np.empty(c.n_leaves, dtype=np.uint64)
    ln = np.empty(c.n_leaves, dtype=np.uint64)
    base = rec_buf.data_ptr()
    for i, (o, n) in enumerate(at_list):
        ptr[i], ln[i] = base + o, n
    for j, obj in enumerate(objs[c.n_s:]):
        ptr[c.n_s + j], ln[c.n_s + j] = obj.data_ptr(), obj.nbytes
    leaf = native.LeafPlan.from_arrays(lib, b"".join(hdrs), hdr_off, hdr_len, hdr_idx, ptr, ln,
                                       np.array(kinds, dtype=np.uint8), dev, fuse=fv)
    fv._keep = []  # the cache keeps nothing of this step's transcript between steps
    k = ctx.k
    buffers = {
        "key": torch.empty(32, dtype=torch.uint8, device=dev),
        "digests": torch.empty(c.n_leaves, 32, dtype=torch.uint8, device=dev),
        "bad": torch.empty(1, dtype=torch.int32, device=dev),
        "rows": torch.empty(c.M, 5 + k, dtype=torch.float64, device=dev),
        "update": torch.empty(max(len(c.linear_weights), 1), 3, dtype=torch.int64, device=dev),
        "side": torch.cuda.Stream(device=dev),
        "h_flags": torch.empty(10, dtype=torch.int32, pin_memory=True),
        "h_digests": torch.empty(c.n_leaves, 32, dtype=torch.uint8, pin_memory=True),
        "h_rows": torch.empty(c.M, 5 + k, dtype=torch.float64, pin_memory=True),
        "h_update": torch.empty(max(len(c.linear_weights), 1), 3, dtype=torch.int64,
                                pin_memory=True),
    }
    return _Entry(leaf_key, fv_key, made, fv, leaf, rec_buf, at_list, bias, None, b"",
                  buffers=buffers)
