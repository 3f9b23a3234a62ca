"""The per-step checks on the hot path, as functions of ``(store, computation, context, bands)``.

Reference: verification/verifier/checks.py:204-251 (``check_2_commitment``), :255-272
(``check_2_root``), :576-658 (``check_5_matmuls``), :866-956 (``_finished``, ``_judge_window``,
``_judge_product``). Each check returns ``None`` on acceptance or a :class:`Rejection`, with
the reference's check ids, rejection kinds and detail strings.

Of the reference's order ``4 → 7 → 2 → 6a → 5 → 6b → 2.root`` this build runs
:data:`DEFAULT_ORDER` = ``2 → 6a → 5 → 2.root``. Checks 4 (batch anchor), 7 (chaining) and 6b
(the glue weights' update identity, which needs the model replay's glue gradients) are not
part of it.

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
- **Check 2's root comparison** runs last and compares the Merkle root over check 2's hashes
  (built on the GPU) with the claimed root.

Operands come from ``c.replay(leaves)``. Rebuilding them by replaying the model is not part of
this build; a computation serves captured operands instead (``DeclaredComputation.
use_operands``).
"""

from __future__ import annotations

import math
from collections.abc import Callable, Iterator
from typing import Any

import torch

from verification.commitment import native
from verification.commitment.leaves import leaf_hashes_of
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
from verification.verifier.matmul_check.freivalds import ProductMeasure, finish_rows

__all__ = ["DEFAULT_ORDER", "ROOT_SLOT", "CHECKS", "protocol_id", "check_2_commitment",
           "check_2_root", "check_6a_linear_update", "check_5_matmuls"]

ROOT_SLOT = "2.root"


def protocol_id(slot: str) -> str:
    """The protocol check id of a slot: ``"2.root"`` rejects as ``"2"``."""
    return slot.split(".", 1)[0]


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
            hashes = leaf_hashes_of(c, read(), ctx.hash_stats())
        stale = any(leaves.changed(i) for i in range(len(leaves)))
        claimed = store.root
    if stale:
        changed = [i for i in range(len(leaves)) if leaves.changed(i)]
        return ctx.reject("2", f"leaf {changed[0]} changed in place during check 2", "malformed")
    for i, h in sorted(ctx.state.early_hashes.items()):
        if hashes[i] != h:
            return ctx.reject("2", f"leaf {i} hashes differently from the bytes an earlier "
                                   f"check read: the store served two versions")
    if not _is_digest(claimed):
        return ctx.reject("2", f"claimed root is not a {DIGEST_SIZE}-byte digest", "malformed")
    changed = [i for i in range(len(leaves)) if leaves.changed(i)]
    if changed:
        return ctx.reject("2", f"leaf {changed[0]} changed in place during check 2", "malformed")
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


@_checked
def check_6a_linear_update(store: TranscriptStore, c: DeclaredComputation, ctx: StepContext,
                           bands: Bands) -> Rejection | None:
    """Check 6 for every linear weight, from its committed weight-gradient leaves
    (checks.py:454-467 with ``_update_identity``, :380-451).

    ``W_t``, ``W_{t+1}`` and the gradient's product leaves are read from check 2's committed
    leaves; one GPU pass over every linear weight gives each weight's ``ρ_max`` (bit for bit
    the reference's), its first non-finite ``R`` or scale and its first ``ρ`` over ``τ_W``.
    The weights are then recorded and judged in declaration order: the first one with a
    non-finite entry, or (when judging) an entry over its band, rejects with the reference's
    wording, and the weights after it are not recorded.
    """
    names = list(c.linear_weights)
    if not names:
        return None
    leaves = ctx.state.committed()
    dev = torch.device("cuda", torch.cuda.current_device())
    with _guard(ctx, "6a", _AFTER_COMMIT):
        weights = []
        for name in names:
            w_t = leaves.leaf(c.w_t_index(name)).to(dev)
            w_next = leaves.leaf(c.w_next_index(name)).to(dev)
            parts = [leaves.leaf(c.product_index(m)).to(dev) for m in c.linear_weights[name]]
            for t in (w_next, *parts):
                if tuple(t.shape) != tuple(w_t.shape):
                    raise RuntimeError(f"{name}: gradient or update of shape {tuple(t.shape)} "
                                       f"!= {tuple(w_t.shape)}")
            weights.append(native.UpdateWeight(w_t.contiguous(), w_next.contiguous(),
                                               [p.contiguous() for p in parts],
                                               bands.tau_w_for(name)))
    with ctx.timed("6a.measure"):
        plan = native.get().update_plan(weights, c.eta, ctx.eps_w)
        try:
            results = native.UpdatePlan.decode(plan.run())
        finally:
            plan.close()
    for name, w, (rho_max, first_nf, first_over) in zip(names, weights, results):
        ctx.stats.tensors.append(TensorStat(name, "6a", rho_max))
        if first_nf is not None:
            r, scale = _entry_values(w, first_nf, c.eta, ctx.eps_w)
            return ctx.reject("6a", f"{name}: entry {first_nf} has a non-finite residual or "
                                    f"bound (|R| = {r:.3e}, scale {scale:.3e})")
        if ctx.judge and first_over is not None:
            r, scale = _entry_values(w, first_over, c.eta, ctx.eps_w)
            tau_w = w.tau_w
            return ctx.reject("6a", f"{name}: entry {first_over} has |R| = {r:.3e}, bound "
                                    f"{tau_w * scale:.3e} (ρ_max = {rho_max:.3g}, "
                                    f"τ_W = {tau_w:g})")
    return None


# ---- check 5: matmuls -------------------------------------------------------------------


def _products(c: DeclaredComputation, leaves: CommittedLeaves, replay: Any
              ) -> list[native.FvProduct]:
    """Every product's ``A``, ``B`` (from the replay), committed ``P`` and, for a biased
    product, its committed ``W_t`` bias in the operand format (as ``[A | 1]·[B ; bᵀ]``), on
    the current GPU (a store may serve host tensors, as the on-disk one does)."""
    dev = torch.device("cuda", torch.cuda.current_device())

    def on_gpu(x: torch.Tensor) -> torch.Tensor:
        return x if x.is_cuda else x.to(dev)

    out = []
    for spec in c.products:
        a, b = (on_gpu(x) for x in replay.operands(spec.m))
        p = on_gpu(leaves.leaf(c.product_index(spec.m)))
        bias = None
        if spec.bias is not None:
            bias = on_gpu(leaves.leaf(c.w_t_index(spec.bias))).to(c.operand_dtype) \
                .to(torch.float32)
        out.append(native.FvProduct(a, b, p, spec.m, bias))
    return out


def check_5_matmuls(store: TranscriptStore, c: DeclaredComputation, ctx: StepContext,
                    bands: Bands) -> Rejection | None:
    """Both tests of check 5 on every product, in canonical order; stop at the first failure.

    The challenges are keyed on ``ctx.state.claimed_root`` (check 2's read validated it).
    Every product is measured at once on the GPU; the rows come back in one read and are
    recorded and judged in canonical order. At a rejection, the products after the failing
    one go to ``StepState.run_rest``, measured and not judged.
    """
    root = ctx.state.claimed_root
    if root is None:
        raise RuntimeError("check 5 needs the claimed root that check 2's read validated")
    leaves = ctx.state.committed()
    with _guard(ctx, "5", _AFTER_COMMIT), ctx.timed("5.glue"):
        replay = c.replay(leaves)
    ctx.state.replay = replay
    if c.M == 0:
        return None
    lib = native.get()
    with _guard(ctx, "5", _AFTER_COMMIT), ctx.timed("5.measure"):
        prods = _products(c, leaves, replay)
        plan = lib.fv_plan(prods, ctx.k, ctx.kappa_guard)
        try:
            rows = plan.rows(root)
            specs = native.verdict_specs(
                [s.q for s in c.products], [s.a_shape[0] for s in c.products],
                [s.bias is not None for s in c.products],
                [bands.kappa_for(product_class(c, s)) for s in c.products], device=rows.device)
            _, _, first = lib.verdicts(rows, specs, k=ctx.k, eps_in=ctx.eps_in,
                                       eps_acc=ctx.eps_acc, tau=bands.tau,
                                       guard=ctx.kappa_guard, judge=ctx.judge)
            host = rows.cpu().numpy()
            device_first = int(first.item())
        finally:
            plan.close()
    with ctx.timed("5.judge"):
        # finish_row on every row at once (the same fp64 operations, bit for bit)
        mps = finish_rows(host, q=[s.q for s in c.products],
                          n=[s.a_shape[0] for s in c.products], eps_in=ctx.eps_in,
                          eps_acc=ctx.eps_acc, guard=ctx.kappa_guard,
                          biased=[s.bias is not None for s in c.products])
        done = list(zip(c.products, mps))
        for i, (spec, mp) in enumerate(done):
            rej = _judge_product(c, spec, mp, ctx, bands)
            if rej is not None:
                if i != device_first:
                    raise RuntimeError(f"check 5: the device verdicts reject product index "
                                       f"{device_first}, the host closed form {i}")
                ctx.state.run_rest = done[i + 1:]
                return rej
    if device_first != c.M:
        raise RuntimeError(f"check 5: the device verdicts reject product index {device_first}, "
                           f"the host closed form accepts every product")
    return None


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
    "2": check_2_commitment,
    "6a": check_6a_linear_update,
    "5": check_5_matmuls,
    ROOT_SLOT: check_2_root,
}
DEFAULT_ORDER: tuple[str, ...] = ("2", "6a", "5", ROOT_SLOT)
