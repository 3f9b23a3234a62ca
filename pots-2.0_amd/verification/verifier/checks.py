"""The per-step checks on the hot path, as functions of ``(store, computation, context, bands)``.

Reference: verification/verifier/checks.py:204-251 (``check_2_commitment``), :255-272
(``check_2_root``), :576-658 (``check_5_matmuls``), :866-956 (``_finished``, ``_judge_window``,
``_judge_product``). Each check returns ``None`` on acceptance or a :class:`Rejection`, with
the reference's check ids, rejection kinds and detail strings.

Of the reference's order ``4 → 7 → 2 → 6a → 5 → 6b → 2.root`` this build runs
:data:`DEFAULT_ORDER` = ``7 → 2 → 6a → 5 → 6b → 2.root``. Check 4 (the batch anchor into
``h_D`` at the schedule's indices) is not part of it.

- **Check 7** (check 0 on the first step) hashes the ``W_t`` leaves on the GPU and compares
  them with the hashes the verifier kept: the agreed ``W_0``'s, or step ``t−1``'s
  ``W_{t+1}``.

- **Check 2's read** reads every leaf once, in order, hashes them on the GPU (through
  ``leaf_hashes_of``, which keeps the first-error-in-order semantics: a malformed or
  non-finite leaf rejects as ``"malformed"`` at check 2), keeps the objects in a
  :class:`CommittedLeaves` reader and validates the claimed root as a digest.
- **Check 5** draws every product's challenges from the claimed root, measures every product
  in one Freivalds plan on the GPU (the three streaming passes, fp64 rows), reads the rows
  back once, then records and judges the products in canonical order on the host exactly as
  the reference does, so the first failing product rejects with the reference's message. The
  device verdict kernel judges the same rows; the two must agree on the first failure.
- **Check 6a** streams every linear weight's ``W_t``, ``W_{t+1}`` and gradient product leaves
  once on the GPU and words the first failing weight's rejection as the reference does.
- **Check 6b** runs the same pass over the glue weights with the gradients check 5's replay
  recomputed through the glue.
- **Check 2's root comparison** runs last and compares the Merkle root over check 2's hashes
  (built on the GPU) with the claimed root.

Operands come from ``c.replay(leaves)``: the MLP instance rebuilds them from the committed
leaves; a computation given the prover's captured operands (``DeclaredComputation.
use_operands``) serves those, which the verifier takes only when trusted, and check 5 marks
the step's statistics with it.
"""

from __future__ import annotations

import math
import weakref
from collections.abc import Callable, Iterator
from typing import Any

import numpy as np
import torch

from verification.commitment import native
from verification.commitment.leaves import leaf_hashes_of, leaf_hashes_until_error
from verification.commitment.merkle import DIGEST_SIZE, merkle_root
from verification.computation.interface import (DeclaredComputation, ProductSpec,
                                                 chain_gradient)
from verification.transcript.store import TranscriptStore
from verification.verifier.bands import Bands, product_class
from verification.verifier.context import (
    _AFTER_COMMIT,
    CommittedLeaves,
    ProductStat,
    Rejection,
    StepContext,
    TensorStat,
    _checked,
    _guard,
    _is_digest,
)
from verification.verifier.matmul_check.freivalds import (ProductMeasure, RowArrays,
                                                           finish_row_arrays)

__all__ = ["DEFAULT_ORDER", "ROOT_SLOT", "CHECKS", "protocol_id", "check_7_chaining",
           "check_2_commitment", "check_2_root", "check_6a_linear_update", "check_5_matmuls",
           "check_6b_glue_update"]

ROOT_SLOT = "2.root"


def protocol_id(slot: str) -> str:
    """The protocol check id of a slot: ``"2.root"`` rejects as ``"2"``."""
    return slot.split(".", 1)[0]


# ---- check 7: chaining (check 0 on the first step) ---------------------------------------


@_checked
def check_7_chaining(store: TranscriptStore, c: DeclaredComputation, ctx: StepContext,
                     bands: Bands) -> Rejection | None:
    """The ``W_t`` leaves hash to the digests the verifier kept: step ``t−1``'s ``W_{t+1}``
    hashes from its check 2, or on the first step the agreed ``W_0``'s, where a mismatch is
    check 0 (reference checks.py:159-197).

    The leaves are read and validated in order and hashed on the GPU, then judged in order:
    the first leaf that fails to read, validate or hash, or that hashes to another digest,
    decides, so an error after a mismatch never shows. Each digest is kept for check 2, which
    must see the same bytes.
    """
    cid = ctx.chain_check_id
    if len(ctx.prev_w_hashes) != c.n_w:
        raise RuntimeError(f"{len(ctx.prev_w_hashes)} chained hashes for {c.n_w} weights")
    read_at = CommittedLeaves()  # versions at read time: a later read may write in place
    slots = [c.w_t_index(name) for name in c.weight_names]

    def read() -> Iterator[tuple[int, Any]]:
        for i in slots:
            obj = store.leaf(i)
            read_at.add(obj)
            yield i, obj

    hashes, error = leaf_hashes_until_error(c, read(), plans=ctx.plans, site="7")
    for pos, got in enumerate(hashes):
        i, name = slots[pos], c.weight_names[pos]
        if read_at.changed(pos):
            return ctx.reject(cid, f"leaf {i} changed in place during check {cid}", "malformed")
        ctx.state.early_hashes[i] = got
        if got != ctx.prev_w_hashes[pos]:
            prior = "the agreed W_0" if cid == "0" else f"W_{{t+1}} of step {ctx.step - 1}"
            return ctx.reject(cid, f"W_t[{name}] differs from {prior}")
    if error is not None:
        with _guard(ctx, cid):
            raise error
    return None


# ---- check 2: commitment ----------------------------------------------------------------


@_checked
def check_2_commitment(store: TranscriptStore, c: DeclaredComputation, ctx: StepContext,
                       bands: Bands) -> Rejection | None:
    """Hash all ``n_leaves`` leaves (the count from ``C``) and validate the claimed ``h``.

    Leaves are read in order and hashed on the GPU; the first malformed leaf (wrong shape or
    dtype, unencodable record, NaN or Inf) rejects as ``"malformed"``, as a leaf-by-leaf loop
    would find it. A leaf that check 4 or 7 read earlier must hash as it did then.
    """
    leaves = CommittedLeaves()

    def read() -> Iterator[tuple[int, Any]]:
        for i in range(c.n_leaves):
            obj = store.leaf(i)
            leaves.add(obj)
            yield i, obj

    with _guard(ctx, "2"):
        with ctx.timed("2.hash"):
            hashes = leaf_hashes_of(c, read(), ctx.hash_stats(), ctx.plans, "2")
        stale = leaves.first_changed()
        claimed = store.root
    if stale is not None:
        return ctx.reject("2", f"leaf {stale} changed in place during check 2", "malformed")
    for i, h in sorted(ctx.state.early_hashes.items()):
        if hashes[i] != h:
            return ctx.reject("2", f"leaf {i} hashes differently from the bytes an earlier "
                                   f"check read: the store served two versions")
    if not _is_digest(claimed):
        return ctx.reject("2", f"claimed root is not a {DIGEST_SIZE}-byte digest", "malformed")
    stale = leaves.first_changed()  # reading the root may have written a leaf
    if stale is not None:
        return ctx.reject("2", f"leaf {stale} changed in place during check 2", "malformed")
    ctx.state.claimed_root, ctx.state.leaf_hashes, ctx.state.leaves = claimed, hashes, leaves
    return None


@_checked
def check_2_root(store: TranscriptStore, c: DeclaredComputation, ctx: StepContext,
                 bands: Bands) -> Rejection | None:
    """The root over check 2's leaf hashes must equal the claimed ``h`` check 5 keyed on."""
    hashes, claimed = ctx.state.leaf_hashes, ctx.state.claimed_root
    if hashes is None or claimed is None:
        raise RuntimeError("check 2's root comparison needs the hashes and claimed root "
                           "of check 2's read")
    root = ctx.state.recomputed_root = merkle_root(hashes)
    if root != claimed:
        return ctx.reject("2", f"recomputed root {root.hex()[:16]}… != claimed "
                               f"{claimed.hex()[:16]}…")
    return None


# ---- check 6a: the update identity of the linear weights -------------------------------


def _entry_values(w: native.UpdateWeight, i: int, eta: float, eps_w: float
                  ) -> tuple[float, float]:
    """``(|R_i|, scale_i)`` of one entry for a rejection's wording, with the reference's fp32
    operations (checks.py:430-432) on that entry alone."""
    one = [x.reshape(-1)[i:i + 1].cpu() for x in (w.w_t, w.w_next)]
    g = chain_gradient([p.reshape(-1)[i:i + 1].cpu() for p in w.parts], torch.float32)
    eta_g = eta * g
    r = (one[1] - (one[0] - eta_g)).abs()
    scale = eps_w * (one[0].abs() + eta_g.abs())
    return float(r), float(scale)


def _update_identity(check_id: str, names: list[str], weights: list[native.UpdateWeight],
                     c: DeclaredComputation, ctx: StepContext) -> Rejection | None:
    """One GPU pass of the update identity over ``weights`` (``ρ_max`` bit for bit the
    reference's, first non-finite ``R`` or scale, first ``ρ`` over ``τ_W``), then recording and
    judging in declaration order with the reference's wording (checks.py:380-467): the first
    weight with a non-finite entry, or (when judging) an entry over its band, rejects, and the
    weights after it are not recorded."""
    with ctx.timed(f"{check_id}.measure"):
        plan = native.get().update_plan(weights, c.eta, ctx.eps_w)
        try:
            results = native.UpdatePlan.decode(plan.run())
        finally:
            plan.close()
    for name, w, (rho_max, first_nf, first_over) in zip(names, weights, results):
        ctx.stats.tensors.append(TensorStat(name, check_id, rho_max))
        if first_nf is not None:
            r, scale = _entry_values(w, first_nf, c.eta, ctx.eps_w)
            return ctx.reject(check_id, f"{name}: entry {first_nf} has a non-finite residual "
                                        f"or bound (|R| = {r:.3e}, scale {scale:.3e})")
        if ctx.judge and first_over is not None:
            r, scale = _entry_values(w, first_over, c.eta, ctx.eps_w)
            tau_w = w.tau_w
            return ctx.reject(check_id, f"{name}: entry {first_over} has |R| = {r:.3e}, bound "
                                        f"{tau_w * scale:.3e} (ρ_max = {rho_max:.3g}, "
                                        f"τ_W = {tau_w:g})")
    return None


def _update_weight(name: str, w_t: torch.Tensor, w_next: torch.Tensor,
                   parts: list[torch.Tensor], tau_w: float) -> native.UpdateWeight:
    dev = torch.device("cuda", torch.cuda.current_device())
    w_t, w_next = w_t.to(dev), w_next.to(dev)
    parts = [p.to(dev) for p in parts]
    for t in (w_next, *parts):
        if tuple(t.shape) != tuple(w_t.shape):
            raise RuntimeError(f"{name}: gradient or update of shape {tuple(t.shape)} "
                               f"!= {tuple(w_t.shape)}")
    return native.UpdateWeight(w_t.contiguous(), w_next.contiguous(),
                               [p.contiguous() for p in parts], tau_w)


@_checked
def check_6a_linear_update(store: TranscriptStore, c: DeclaredComputation, ctx: StepContext,
                           bands: Bands) -> Rejection | None:
    """Check 6 for every linear weight, from its committed weight-gradient leaves
    (checks.py:454-467 with ``_update_identity``, :380-451).

    ``W_t``, ``W_{t+1}`` and the gradient's product leaves are read from check 2's committed
    leaves; one GPU pass over every linear weight gives each weight's ``ρ_max`` (bit for bit
    the reference's), its first non-finite ``R`` or scale and its first ``ρ`` over ``τ_W``.
    """
    names = list(c.linear_weights)
    if not names:
        return None
    leaves = ctx.state.committed()
    with _guard(ctx, "6a", _AFTER_COMMIT):
        weights = [_update_weight(name, leaves.leaf(c.w_t_index(name)),
                                  leaves.leaf(c.w_next_index(name)),
                                  [leaves.leaf(c.product_index(m))
                                   for m in c.linear_weights[name]], bands.tau_w_for(name))
                   for name in names]
    return _update_identity("6a", names, weights, c, ctx)


# ---- check 6b: the update identity of the glue weights ----------------------------------


@_checked
def check_6b_glue_update(store: TranscriptStore, c: DeclaredComputation, ctx: StepContext,
                         bands: Bands) -> Rejection | None:
    """Check 6 for every glue weight (the norms' γ, the biases, the tied embedding), with the
    gradient check 5's replay recomputed through the glue (reference checks.py:960-995).

    The gradient is the replay's, in fp32; ``W_t`` and ``W_{t+1}`` are check 2's committed
    leaves; the identity, its ``ρ_max`` and its wording are check 6a's. A replay of the prover's
    captured operands has no glue to recompute: the step's statistics already say check 5
    measured the prover's operands, and 6b is not run.
    """
    names = list(c.glue_gradient_weights)
    if not names:
        return None
    replay = ctx.state.replay
    if replay is None:
        raise RuntimeError("check 6b needs check 5's replay")
    if getattr(replay, "prover_supplied", False):
        return None
    with _guard(ctx, "6b", _AFTER_COMMIT), ctx.timed("6b.glue"):
        grads = replay.glue_gradients()
    missing = [name for name in names if name not in grads]
    if missing:
        raise RuntimeError(f"the replay returned no glue gradient for {missing}")
    leaves = ctx.state.committed()
    with _guard(ctx, "6b", _AFTER_COMMIT):
        weights = [_update_weight(name, leaves.leaf(c.w_t_index(name)),
                                  leaves.leaf(c.w_next_index(name)),
                                  [grads[name].detach().to(torch.float32)],
                                  bands.tau_w_for(name))
                   for name in names]
    return _update_identity("6b", names, weights, c, ctx)


# ---- check 5: matmuls -------------------------------------------------------------------


def _serve_until_error(c: DeclaredComputation, ctx: StepContext, leaves: CommittedLeaves,
                       replay: Any) -> tuple[list[native.FvProduct], Exception | None]:
    """Every product served in canonical order, up to the first whose serving raises: the
    products before it and that error (``None`` when all are served).

    Product ``m`` is its ``A``, ``B`` from the replay, its committed ``P`` and, for a biased
    product, its committed ``W_t`` bias in the operand format (as ``[A | 1]·[B ; bᵀ]``), on
    the current GPU (a store may serve host tensors, as the on-disk one does). A prover-data
    error while serving is check 5's malformed rejection; operands of the wrong shape are a
    verifier error (reference checks.py:805-833). Either is returned, to be raised after the
    products before it are judged."""
    def dev() -> torch.device:
        return torch.device("cuda", torch.cuda.current_device())

    operands = replay.operands
    timed = ctx.section is not None
    p_base = c.n_s + c.n_w - 1
    out: list[native.FvProduct] = []
    for spec in c.products:
        try:
            try:
                if timed:
                    with ctx.timed("5.glue"):
                        a, b = operands(spec.m)
                else:
                    a, b = operands(spec.m)
                p = leaves.leaf(p_base + spec.m)
                bias = None
                if spec.bias is not None:
                    bias = leaves.leaf(c.w_t_index(spec.bias)).to(dev()) \
                        .to(c.operand_dtype).to(torch.float32)
            except _AFTER_COMMIT as e:  # prover data: check 5's malformed rejection
                with _guard(ctx, "5", _AFTER_COMMIT):
                    raise e
            if a.shape != spec.a_shape or b.shape != spec.b_shape:
                raise RuntimeError(f"{spec.name}: replay operands {tuple(a.shape)}·"
                                   f"{tuple(b.shape)} != declared {spec.a_shape}·{spec.b_shape}")
            if not a.is_cuda:
                a = a.to(dev())
            if not b.is_cuda:
                b = b.to(dev())
            if not p.is_cuda:
                p = p.to(dev())
            out.append(native.FvProduct(a, b, p, spec.m, bias))
        except Exception as e:  # judged after the products before it
            return out, e
    return out, None


_PRODUCT_TABLES: weakref.WeakKeyDictionary[Any, tuple[list[str], np.ndarray, np.ndarray,
                                                      np.ndarray]] = weakref.WeakKeyDictionary()


def _product_table(c: DeclaredComputation) -> tuple[list[str], np.ndarray, np.ndarray,
                                                    np.ndarray]:
    """Per product in canonical order: its κ class, ``q``, ``n`` and whether it is biased;
    built once per computation (its layout does not change)."""
    try:
        table = _PRODUCT_TABLES.get(c)
    except TypeError:
        table = None
    if table is None or len(table[0]) != c.M:
        table = ([product_class(c, s) for s in c.products],
                 np.array([s.q for s in c.products], dtype=np.int64),
                 np.array([s.a_shape[0] for s in c.products], dtype=np.int64),
                 np.array([s.bias is not None for s in c.products], dtype=bool))
        try:
            _PRODUCT_TABLES[c] = table
        except TypeError:
            pass
    return table


def _first_rejected(f: RowArrays, kappa_max: np.ndarray, ctx: StepContext,
                    bands: Bands) -> int:
    """The index of the first product :func:`_judge_product` rejects, or ``M``: the same
    tests on arrays (finiteness of what is judged; then, when judging, ``ν ≤ κ_max·‖|P|·1‖``
    and every residual ``≤ τ·unit``, where NaN fails)."""
    bad = ~(np.isfinite(f.p_norm) & np.isfinite(f.u) & np.isfinite(f.unit)
            & np.isfinite(f.residuals).all(axis=1))
    if ctx.kappa_guard:
        bad |= ~(np.isfinite(f.nu) & np.isfinite(f.p_abs1))
    if ctx.judge:
        with np.errstate(invalid="ignore", over="ignore"):
            if ctx.kappa_guard:
                bad |= ~(f.nu <= kappa_max * f.p_abs1)
            bad |= ~(f.residuals <= bands.tau * f.unit[:, None]).all(axis=1)
    hit = np.flatnonzero(bad)
    return int(hit[0]) if hit.size else len(bad)


def _measure_and_judge(c: DeclaredComputation, prods: list[native.FvProduct], root: bytes,
                       ctx: StepContext, bands: Bands) -> Rejection | None:
    """Measure ``prods`` (the first ``len(prods)`` products in canonical order) in one
    Freivalds plan, read the rows back once, then record and judge them in order; the device
    verdict kernel judges the same rows and must agree on the first failure.

    Judging is the reference's per-product closed form and tests (``finish_row``,
    ``_judge_product``) evaluated on arrays, with the same IEEE operations; the first
    rejected product is then judged on its own, which words its rejection."""
    n = len(prods)
    specs = c.products[:n]
    if not specs:
        return None
    classes, qs, ns, biased = _product_table(c)
    qs, ns, biased = qs[:n], ns[:n], biased[:n]
    kappa_of = {cls: bands.kappa_for(cls) for cls in set(classes[:n])}
    kappa_max = np.array([kappa_of[cls] for cls in classes[:n]], dtype=np.float64)
    lib = native.get()
    with ctx.timed("5.measure"):
        cache = ctx.plans
        plan = cache.fv_plan(prods, ctx.k, ctx.kappa_guard) if cache is not None \
            else lib.fv_plan(prods, ctx.k, ctx.kappa_guard)
        try:
            rows = plan.rows(root)
            vspecs = native.verdict_specs(qs, ns, biased, kappa_max, device=rows.device)
            _, _, first = lib.verdicts(rows, vspecs, k=ctx.k, eps_in=ctx.eps_in,
                                       eps_acc=ctx.eps_acc, tau=bands.tau,
                                       guard=ctx.kappa_guard, judge=ctx.judge)
            host = rows.cpu().numpy()
            device_first = int(first.item())
        finally:
            if cache is not None:
                cache.release(plan)
            else:
                plan.close()
    with ctx.timed("5.judge"):
        return judge_rows(c, host, device_first, kappa_max, ctx, bands)


def judge_rows(c: DeclaredComputation, host: np.ndarray, device_first: int,
               kappa_max: np.ndarray, ctx: StepContext, bands: Bands) -> Rejection | None:
    """Record and judge the measured rows of the first ``len(host)`` products in canonical
    order (``kappa_max`` per product); the device verdicts' first rejected index must agree.
    At a rejection, the products after the failing one go to ``StepState.run_rest``."""
    n = len(host)
    specs = c.products[:n]
    classes, qs, ns, biased = _product_table(c)
    qs, ns, biased = qs[:n], ns[:n], biased[:n]
    f = finish_row_arrays(host, q=qs, n=ns, eps_in=ctx.eps_in, eps_acc=ctx.eps_acc,
                          guard=ctx.kappa_guard, biased=biased)
    stop = _first_rejected(f, kappa_max, ctx, bands)
    if stop != device_first:
        raise RuntimeError(f"check 5: the device verdicts reject product index "
                           f"{device_first}, the host closed form {stop}")
    def made(f=f, stop=stop) -> Iterator[ProductStat]:
        cols = (f.kappa[:stop].tolist(), f.normalized[:stop].tolist(),
                f.p_norm[:stop].tolist(), f.nu[:stop].tolist(), f.p_abs1[:stop].tolist(),
                f.u[:stop].tolist())
        return (ProductStat(s.m, s.name, cls, kp, tuple(nz), s.q, pn, nu, pa, uu)
                for s, cls, kp, nz, pn, nu, pa, uu in zip(specs[:stop], classes, *cols))

    ctx.stats.add_products(made)  # made into records when first read
    if stop == n:
        return None
    rej = _judge_product(c, specs[stop], f.measure(stop), ctx, bands)
    if rej is None:
        raise RuntimeError(f"check 5: product index {stop} fails the array tests but "
                           f"not the per-product judge")
    ctx.state.run_rest = [(s, f.measure(i)) for i, s in enumerate(specs[stop + 1:],
                                                                  start=stop + 1)]
    return rej


@_checked
def check_5_matmuls(store: TranscriptStore, c: DeclaredComputation, ctx: StepContext,
                    bands: Bands) -> Rejection | None:
    """Both tests of check 5 on every product, in canonical order; stop at the first failure.

    The challenges are keyed on ``ctx.state.claimed_root`` (check 2's read validated it).
    The products are served in canonical order, every one measured at once on the GPU; the
    rows come back in one read and are recorded and judged in canonical order. At a
    rejection, the products after the failing one go to ``StepState.run_rest``, measured and
    not judged.

    An error while serving product ``m`` is raised only after the products before ``m`` are
    judged, as it would be one product at a time (reference checks.py:613-650): if one of them
    rejects, that rejection is returned and the error goes to ``StepState.run_rest_error``;
    otherwise the error is raised, and a prover-data error becomes check 5's malformed
    rejection.
    """
    root = ctx.state.claimed_root
    if root is None:
        raise RuntimeError("check 5 needs the claimed root that check 2's read validated")
    leaves = ctx.state.committed()
    with _guard(ctx, "5", _AFTER_COMMIT), ctx.timed("5.glue"):
        replay = c.replay(leaves)
    ctx.state.replay = replay
    if getattr(replay, "prover_supplied", False):
        if not ctx.trust_prover_operands:
            raise RuntimeError("check 5 was given the prover's captured operands without "
                               "trust_prover_operands")
        ctx.stats.operands_from_prover = True
    if c.M == 0:
        return None
    prods, error = _serve_until_error(c, ctx, leaves, replay)
    rej = _measure_and_judge(c, prods, root, ctx, bands)
    if error is None:
        return rej
    if rej is None:
        raise error
    ctx.state.run_rest_error = error
    return rej


def _judge_product(c: DeclaredComputation, spec: ProductSpec, mp: ProductMeasure,
                   ctx: StepContext, bands: Bands) -> Rejection | None:
    """Record product ``spec.m``'s numbers, then judge them: finiteness, test 1, test 2."""
    cls_key = product_class(c, spec)
    nu, p_abs1, kappa, res, unit = mp.nu, mp.p_abs1, mp.kappa, mp.residuals, mp.unit
    normalized = mp.normalized
    ctx.stats.products.append(ProductStat(spec.m, spec.name, cls_key, kappa, normalized,
                                          q=spec.q, p_norm=mp.p_norm, nu=nu,
                                          p_abs1=p_abs1, u=mp.u))
    guard = {"ν": nu, "‖|P|·1‖": p_abs1} if ctx.kappa_guard else {}
    values = {**guard, "‖P‖_F": mp.p_norm, "U": mp.u, "band unit": unit,
              **{f"residual j={j}": x for j, x in enumerate(res, start=1)}}
    bad = [key for key, v in values.items() if not math.isfinite(v)]
    if bad:
        return ctx.reject("5", f"P_{spec.m} ({spec.name}): non-finite {', '.join(bad)}")
    if not ctx.judge:
        return None
    kappa_max = bands.kappa_for(cls_key)
    if ctx.kappa_guard and not nu <= kappa_max * p_abs1:
        return ctx.reject("5", f"P_{spec.m} ({spec.name}): cancellation factor κ = "
                               f"{kappa:.3g} > κ_max = {kappa_max:g} [{cls_key}]")
    for j, x in enumerate(res, start=1):
        if not x <= bands.tau * unit:
            return ctx.reject("5", f"P_{spec.m} ({spec.name}), challenge j={j}: normalized "
                                   f"residual {normalized[j - 1]:.3g} > τ = {bands.tau:g}")
    return None


CHECKS: dict[str, Callable[..., Rejection | None]] = {
    "7": check_7_chaining,
    "2": check_2_commitment,
    "6a": check_6a_linear_update,
    "5": check_5_matmuls,
    "6b": check_6b_glue_update,
    ROOT_SLOT: check_2_root,
}
DEFAULT_ORDER: tuple[str, ...] = ("7", "2", "6a", "5", "6b", ROOT_SLOT)
