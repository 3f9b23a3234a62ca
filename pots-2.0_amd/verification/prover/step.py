"""One honest SGD step under capture, committed on the GPU (reference:
verification/prover/step.py:61-269, ``StepOutput``, ``prove_step``, ``commit``).

:func:`prove_step` runs ``C(b, W_t)``: the training pass under :class:`MatmulCapture`, the
labeling into canonical slots, the version guard, then plain SGD at the declared ``eta``. It
returns a :class:`StepOutput` holding the leaves in transcript order. :func:`commit` builds the
step's Merkle tree.

The difference from the reference is where the transcript lives. The reference copies every
captured product to pinned host memory as it is produced and hashes the leaves on the host.
Here the products stay in the device memory the model computed them in, ``W_t`` and
``W_{t+1}`` are device copies, and :func:`commit` hashes every leaf in place with the same
kernels the verifier uses (``commit_leaves_device``: the chunk kernel, the per-leaf trees and
the outer tree), reading the records from the host. Nothing but the 32-byte digests crosses
PCIe.
"""

from __future__ import annotations

from collections.abc import Callable, Iterator, Mapping, Sequence
from contextlib import contextmanager
from dataclasses import dataclass, field
from typing import Any

import torch

from verification.computation.interface import (DeclaredComputation, load_weights,
                                               snapshot_weights)
from verification.computation.matmul_ops import param_storage_map
from verification.prover.capture import MatmulCapture, MutatedCaptureError

__all__ = ["StepOutput", "prove_step", "commit"]

Perturbation = Callable[[torch.Tensor], torch.Tensor]


def _versions(objs: Sequence[Any]) -> tuple[int, ...]:
    out: list[int] = []
    for o in objs:
        if isinstance(o, torch.Tensor):
            out.append(o._version)
        else:  # a record of several tensors
            out.extend(t._version for t in (o.ids, o.targets, o.mask))
    return tuple(out)


@dataclass(frozen=True, eq=False)
class StepOutput:
    """One proved step: the leaves ``[records | W_t | P_1..P_M | W_{t+1}]`` and the versions
    of every leaf tensor when the step was emitted."""

    records: tuple[Any, ...]
    w_t: dict[str, torch.Tensor]
    products: tuple[torch.Tensor, ...]
    w_next: dict[str, torch.Tensor]
    loss: float
    versions: tuple[int, ...] = field(repr=False)
    capture: dict = field(default_factory=dict, repr=False)
    # {m: (A_m, B_m)} as captured, when prove_step was asked to keep them
    operands: dict = field(default_factory=dict, repr=False)

    def replay(self):
        """The kept operands as check 5's operand source."""
        from verification.prover.synthetic import CapturedReplay
        return CapturedReplay(self.operands)

    def leaves(self) -> list[Any]:
        return [*self.records, *self.w_t.values(), *self.products, *self.w_next.values()]

    def assert_unmodified(self) -> None:
        """Raise :class:`MutatedCaptureError` if any leaf was written in place since the step
        was emitted (invariant 6)."""
        if _versions(self.leaves()) != self.versions:
            raise MutatedCaptureError("a leaf of the step was written in place after the step")


def _w_t_leaves(c: DeclaredComputation, model: torch.nn.Module,
                w_t: Mapping[str, torch.Tensor]) -> dict[str, torch.Tensor]:
    """The committed ``W_t``: the caller's tensor where it can be shared (contiguous, the
    model's dtype, shape and device, owning its storage, no grad, not a parameter's storage),
    else a copy of the loaded parameter (reference step.py:115-139)."""
    model_storages = {p.untyped_storage().data_ptr() for p in model.parameters()}
    out = {}
    for name in c.weight_names:
        p, w = model.get_parameter(name), w_t[name]
        share = (w.is_contiguous() and w.dtype == p.dtype and w.shape == p.shape
                 and w.device == p.device and not w.requires_grad and w.storage_offset() == 0
                 and w.untyped_storage().nbytes() == w.numel() * w.element_size()
                 and w.untyped_storage().data_ptr() not in model_storages)
        out[name] = w if share else p.detach().clone()
    return out


def prove_step(c: DeclaredComputation, model: torch.nn.Module, w_t: Mapping[str, torch.Tensor],
               records: Sequence[Any], *, perturb: Mapping[int, Perturbation] | None = None,
               keep_operands: bool = False) -> StepOutput:
    """Run ``C(b, W_t)`` on ``model`` and emit the step's leaves.

    ``model`` is loaded with ``w_t`` and left holding ``W_{t+1}`` with its gradients cleared.
    ``perturb`` (``{m: fn}``) replaces committed product ``P_m`` by ``fn(copy of P_m)`` after
    the capture, a prover-side cheat for tests; training uses the true gradients.
    ``keep_operands`` keeps every product's captured ``(A_m, B_m)`` (the computation's
    ``label_with_operands``), for a computation whose replay is not built.
    """
    if len(records) != c.n_s:
        raise ValueError(f"batch has {len(records)} records, the computation declares {c.n_s}")
    if not torch.is_grad_enabled():
        raise RuntimeError("prove_step needs grad mode on")
    record_versions = _versions(records)
    load_weights(c, model, w_t)
    w_t_leaves = _w_t_leaves(c, model, w_t)
    w_t_versions = _versions(list(w_t_leaves.values()))
    model.zero_grad(set_to_none=True)
    opt = torch.optim.SGD(model.parameters(), lr=c.eta)

    cap = MatmulCapture(param_names=param_storage_map(model))

    @contextmanager
    def stage(p: str) -> Iterator[None]:
        with cap.phase(p):
            yield

    with cap:
        loss = c.forward_backward(model, records, stage)
    operands: dict = {}
    if keep_operands:
        labeled, captured = c.label_with_operands(cap, model)

        def held(t: torch.Tensor) -> torch.Tensor:
            # An operand that views a parameter (a linear's W.t(), an input gradient's W)
            # would see the SGD step: it is served from the committed W_t leaf instead. A
            # copy of a parameter (autocast's bf16 weight) is a tensor of its own.
            name = cap.param_names.get(t.untyped_storage().data_ptr())
            if name is not None and name in w_t_leaves:
                return w_t_leaves[name].as_strided(t.shape, t.stride(), t.storage_offset())
            return t.detach()

        operands = {m: (held(a), held(b)) for m, (a, b) in captured.items()}
    else:
        labeled = c.label(cap, model)
    products = [p.detach() for p in labeled]
    if len(products) != c.M:
        raise RuntimeError(f"label returned {len(products)} products, M = {c.M}")
    cap.assert_unmodified()
    product_versions = list(_versions(products))
    cap.release_operands()
    summary = cap.summary()

    for m, fn in (perturb or {}).items():
        spec = c.product(m)
        new = fn(products[m - 1].clone())
        if tuple(new.shape) != spec.p_shape or new.dtype != products[m - 1].dtype:
            raise ValueError(f"perturbation of {spec.name} changed its shape or dtype")
        products[m - 1] = new.detach().contiguous()
        product_versions[m - 1] = products[m - 1]._version

    opt.step()
    w_next = snapshot_weights(c, model)
    # set_to_none drops the model's reference to the gradients; the G products stay intact.
    model.zero_grad(set_to_none=True)
    return StepOutput(
        records=tuple(records), w_t=w_t_leaves, products=tuple(products), w_next=w_next,
        loss=float(loss.detach()),
        versions=(record_versions + w_t_versions + tuple(product_versions)
                  + _versions(list(w_next.values()))),
        capture=summary, operands=operands)


def commit(c: DeclaredComputation, step: StepOutput):
    """The Merkle tree over the step's leaves, hashed on the GPU where they lie; ``.root`` is
    ``h`` (reference step.py:265-269)."""
    from verification.commitment.leaves import commit_leaves_device
    tree = commit_leaves_device(c, step.leaves())
    step.assert_unmodified()  # nothing moved while it was hashed
    return tree
