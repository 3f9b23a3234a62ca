"""A training pass with every checked product taken from its committed leaf (the verifier's
replay; reference: verification/computation/substitution.py:59, ``ProductSubstitution``, and
instances/decoder.py:1142-1751, ``DecoderReplay``).

The verifier rebuilds check 5's operands ``A_m, B_m`` by running the model's own code on the
committed batch and ``W_t``, so that everything between products (norms, softmax, RoPE,
activations, residual sums, the loss and autograd's glue) is recomputed from committed values
and every product is the leaf the prover committed. Two passes do it:

1. **The plan.** One training pass under :class:`~verification.prover.capture.MatmulCapture`, labeled by the computation's own ``label_with_operands``, gives for every
   matmul call of a pass (counted in dispatch order, outer products included) the product
   slots its output fills: one slot, or one per member of a batched call, and whether the slot
   holds the member's output transposed. The call sequence of a pass depends on the model's
   code and the shapes only, never on the values, so the plan holds for any step of ``C``.
2. **The replay.** The same pass under :class:`CommittedProducts`: each planned call returns
   its slots' committed leaves (a copy; a batched call's members stacked, a transposed slot
   transposed back) instead of computing, and keeps the operands it received as the slots'
   ``(A, B)``; a call the plan does not cover (an outer product, glue) runs as it is. A call
   that does not match the plan (another op or output shape) raises :class:`ReplayError`.

The replay's backward leaves each weight's full gradient in ``.grad``: for a glue weight
(a norm's γ, a bias, the embedding) that is check 6b's ``G``, recomputed from committed
products through the glue.
"""

from __future__ import annotations

import contextlib
from collections.abc import Callable, Iterator, Sequence
from dataclasses import dataclass
from typing import Any

import torch
from torch.utils._python_dispatch import TorchDispatchMode

from verification.computation.matmul_ops import HANDLED_OPS, param_storage_map
from verification.prover.capture import MatmulCapture

__all__ = ["ReplayError", "CallPlan", "plan_calls", "CommittedProducts"]

# slot fills of one call: (member index or None, slot name, transposed)
Fill = tuple[int | None, str, bool]


class ReplayError(RuntimeError):
    """The replayed pass departs from the plan: a verifier-side bug, not prover data."""


@dataclass(frozen=True)
class CallPlan:
    """What each matmul call of a training pass of ``C`` fills: ``fills[i]`` for call ``i``
    (absent for glue calls), ``ops[i]`` its op and output shape, ``n_calls`` the calls in
    all."""

    fills: dict[int, list[Fill]]
    ops: dict[int, tuple[str, tuple[int, ...]]]
    n_calls: int


def plan_calls(c: Any, model: torch.nn.Module, records: Sequence[Any]) -> CallPlan:
    """The plan, from one recorded training pass of ``model`` on ``records`` labeled by
    ``c.label_with_operands``. The pass's own products are the verifier's, used only to tell
    the calls apart; the model's gradients are cleared afterwards."""
    cap = MatmulCapture(param_names=param_storage_map(model))
    model.zero_grad(set_to_none=True)
    with torch.enable_grad(), cap:
        c.forward_backward(model, records, cap.phase)
    fills: dict[int, list[Fill]] = {}
    c.label_with_operands(cap, model, call_slots=fills)
    ops = {rec.index: (rec.op, tuple(rec.out.shape)) for rec in cap.records}
    n_calls = len(cap.records) + len(cap.glue_outer)
    model.zero_grad(set_to_none=True)
    return CallPlan(fills, ops, n_calls)


class CommittedProducts(TorchDispatchMode):
    """The replay pass's dispatch mode: a planned call returns its committed products and
    records its operands (``held[slot] = (A, B, A._version, B._version)``)."""

    def __init__(self, plan: CallPlan, leaf: Callable[[str], torch.Tensor]) -> None:
        super().__init__()
        self.plan, self.leaf = plan, leaf
        self.held: dict[str, tuple[torch.Tensor, torch.Tensor, int, int]] = {}
        # each batched call's whole operands, by its first member's slot: (its members' slots
        # in batch order, A, B, their versions, whether the slots hold the members transposed)
        self.batched: dict[str, tuple[tuple[str, ...], torch.Tensor, torch.Tensor, int, int,
                                      bool]] = {}
        self.calls = 0
        self._phase: str | None = None

    @contextlib.contextmanager
    def phase(self, name: str) -> Iterator[None]:
        if self._phase is not None:
            raise ReplayError(f"phase {name!r} entered inside {self._phase!r}")
        self._phase = name
        try:
            yield
        finally:
            self._phase = None

    def _keep(self, slot: str, a: torch.Tensor, b: torch.Tensor) -> None:
        if slot in self.held:
            raise ReplayError(f"slot {slot} filled twice")
        a, b = a.detach(), b.detach()
        self.held[slot] = (a, b, a._version, b._version)

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        name = func.overloadpacket.__name__
        if func.namespace != "aten" or name not in HANDLED_OPS:
            return func(*args, **kwargs)
        if self._phase is None:
            raise ReplayError(f"{func} ran outside the replay's phases")
        index = self.calls
        self.calls += 1
        fills = self.plan.fills.get(index)
        if fills is None:  # glue: an outer product runs as it is
            return func(*args, **kwargs)
        op, shape = self.plan.ops[index]
        if str(func) != op:
            raise ReplayError(f"call {index} is {func}; the plan has {op}")
        a, b = (args[1], args[2]) if name in ("addmm", "baddbmm") else (args[0], args[1])
        if name in ("bmm", "baddbmm"):
            members: list[torch.Tensor | None] = [None] * a.shape[0]
            for i, slot, transposed in fills:
                p = self.leaf(slot)
                members[i] = p.transpose(0, 1) if transposed else p
                if transposed:  # the slot's product is the member's output transposed
                    self._keep(slot, b[i].transpose(0, 1), a[i].transpose(0, 1))
                else:
                    self._keep(slot, a[i], b[i])
            if any(p is None for p in members):
                raise ReplayError(f"call {index}: the plan leaves members unfilled")
            order = sorted(fills, key=lambda f: f[0])
            flips = {f[2] for f in order}
            if len(flips) == 1:
                wa, wb = a.detach(), b.detach()
                self.batched[order[0][1]] = (tuple(f[1] for f in order), wa, wb, wa._version,
                                             wb._version, flips.pop())
            out = torch.stack(members)
        else:
            if len(fills) != 1 or fills[0][0] is not None:
                raise ReplayError(f"call {index}: a plain product with {len(fills)} slots")
            slot = fills[0][1]
            out = self.leaf(slot).clone()
            self._keep(slot, a, b)
        if tuple(out.shape) != shape or out.dtype != a.dtype or out.device != a.device:
            raise ReplayError(f"call {index} ({op}): committed {out.dtype} "
                              f"{tuple(out.shape)} on {out.device} for an output of "
                              f"{a.dtype} {shape} on {a.device}")
        return out
