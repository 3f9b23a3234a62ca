"""Recording every matmul of a forward and backward pass, with the products kept in HBM
(reference: verification/prover/capture.py:1-602, ``MatmulCapture``).

The prover captures its training step with it (``verification.prover.capture`` re-exports
it), and the verifier's decoder replay runs it once to learn which call of a pass fills which
product slot; it holds no prover state.

Wrap a model's forward pass and ``loss.backward()`` in a :class:`MatmulCapture`; every
matmul-family aten op that reaches dispatch is recorded with its operands as the op received
them and its real output, and the op's own result is returned, so training is unchanged:

    cap = MatmulCapture(param_names=param_storage_map(model))
    with cap:
        with cap.phase("forward"):
            loss = loss_fn(model(x), y)
        with cap.phase("backward"):
            loss.backward()
    cap.assert_unmodified()

The recording rules are the reference's:

- ``aten.mm`` and ``aten.bmm`` give one :class:`MatmulRecord`; each member ``A[i]·B[i]`` of a
  ``bmm`` is a checked product of its own.
- ``aten.addmm`` and ``aten.baddbmm`` are accepted with ``alpha == 1`` when the bias term is
  inert (``beta == 0`` or an all-zero bias), and ``addmm`` also in the bias rule's form: a
  vector of length ``b.shape[1]`` added once (``beta == 1``), kept as the record's ``bias``.
  Any other bias raises :class:`BiasedMatmulError`.
- A product with contracted length ``q = 1`` is an outer product, glue: it goes to
  :attr:`MatmulCapture.glue_outer`.
- A refused op (``REJECTED_OPS``), a non-default overload of a handled op, or, inside a phase,
  an op outside the ``aten`` and ``prims`` namespaces that ``ALLOWED_NAMESPACE_OPS`` does not
  list raises :class:`UnsupportedMatmulError`; a handled op outside a phase raises
  :class:`PhaseError`.
- ``aten._to_copy`` inside a phase gives a :class:`CopyRecord`. A copy of a parameter (such as
  autocast's bf16 weight) is held until :meth:`release_operands` and marks the operands that
  alias it (:attr:`OperandInfo.param_copy`); other copies are tracked through a weak reference
  to their storage only, so the capture keeps no activation alive.

**Where the products live.** The reference copies each GPU output to a pinned host buffer on a
side stream as soon as the op returns, so the transcript collects in host RAM, and hashes it
there. On an MI355X the whole step's products fit in HBM (a Qwen2-1.5B-shaped step's 50 GB
against 288 GB), and the leaf hasher reads them where they lie. So a record's ``out`` stays the
op's own output, on the device that computed it, and nothing is copied: no device-to-host
traffic during the step and none for the commit. Invariant 6 holds through the version guard:
:meth:`assert_unmodified` compares every captured tensor's ``_version`` with the value seen at
capture (writes that bypass autograd's bookkeeping are not seen, as in the reference).
"""

from __future__ import annotations

import contextlib
from collections import Counter
from collections.abc import Iterator, Mapping
from dataclasses import dataclass, field

import torch
from torch.multiprocessing.reductions import StorageWeakRef
from torch.utils._python_dispatch import TorchDispatchMode

from verification.computation.matmul_ops import (ALLOWED_NAMESPACE_OPS, HANDLED_OPS,
                                                 REJECTED_OPS, TRUSTED_NAMESPACES)

__all__ = ["PHASES", "CaptureError", "UnsupportedMatmulError", "BiasedMatmulError",
           "PhaseError", "MutatedCaptureError", "OperandInfo", "MatmulRecord", "CopyRecord",
           "MatmulCapture"]

PHASES = ("forward", "backward")

# name -> (batched, takes a bias term)
_FORMS = {"mm": (False, False), "bmm": (True, False), "addmm": (False, True),
          "baddbmm": (True, True)}
assert frozenset(_FORMS) == HANDLED_OPS
_TO_COPY = torch.ops.aten._to_copy.default


class CaptureError(RuntimeError):
    """The step cannot be captured as the declared computation needs it."""


class UnsupportedMatmulError(CaptureError):
    """A matrix product reached dispatch in a form the capture does not record."""


class BiasedMatmulError(CaptureError):
    """An addmm/baddbmm whose bias term the bias rule does not cover."""


class PhaseError(CaptureError):
    """A product ran outside a phase, or phases were nested."""


class MutatedCaptureError(CaptureError):
    """A captured tensor was written in place after it was captured."""


@dataclass(frozen=True)
class OperandInfo:
    """Identity of a captured tensor for labeling. ``storage_ptr`` is meaningful while the
    capture holds the tensor; ``producer_index`` is the index of the earlier record whose
    output storage it aliases (``None`` for glue or a parameter) and stays valid after
    :meth:`MatmulCapture.release_operands`; ``param_copy`` names the parameter when the tensor
    aliases a ``_to_copy`` of it."""

    storage_ptr: int
    storage_offset: int
    shape: tuple[int, ...]
    stride: tuple[int, ...]
    dtype: torch.dtype
    param_name: str | None
    producer_index: int | None = None
    param_copy: str | None = None


@dataclass
class MatmulRecord:
    """One captured matmul call: ``a``, ``b`` (``None`` after ``release_operands``) and the
    op's output ``out``, in device memory where the op ran."""

    index: int          # call index among all matmul-family calls, checked and glue
    op: str             # e.g. "aten.mm.default"
    phase: str
    a: torch.Tensor | None
    b: torch.Tensor | None
    out: torch.Tensor
    q: int              # contracted length
    batch: int | None   # bmm/baddbmm batch size, else None
    a_info: OperandInfo
    b_info: OperandInfo
    out_info: OperandInfo
    bias: torch.Tensor | None = None
    alpha: float = 1.0
    beta: float = 1.0
    versions: dict[str, int] = field(default_factory=dict, repr=False)
    out_storage: StorageWeakRef | None = field(default=None, repr=False, compare=False)

    @property
    def n_members(self) -> int:
        return 1 if self.batch is None else self.batch

    def tensors(self) -> dict[str, torch.Tensor]:
        held = {"a": self.a, "b": self.b, "out": self.out, "bias": self.bias}
        return {k: t for k, t in held.items() if t is not None}

    def members(self) -> Iterator[tuple[torch.Tensor, torch.Tensor, torch.Tensor]]:
        """``(A_i, B_i, P_i)`` per checked product."""
        if self.a is None or self.b is None:
            raise CaptureError(f"record #{self.index}: operands were released")
        if self.batch is None:
            yield self.a, self.b, self.out
            return
        for i in range(self.batch):
            yield self.a[i], self.b[i], self.out[i]


@dataclass
class CopyRecord:
    """One ``aten._to_copy`` inside a phase; ``storage`` is a weak reference to the output's
    storage (its identity, not its memory)."""

    index: int
    phase: str
    src_info: OperandInfo
    out_info: OperandInfo
    storage: StorageWeakRef = field(repr=False)

    @property
    def param(self) -> str | None:
        """The parameter this copies, directly or through earlier copies."""
        return self.src_info.param_name or self.src_info.param_copy


class MatmulCapture(TorchDispatchMode):
    """A passthrough dispatch mode that records every matmul of a forward and backward pass,
    keeping the products where the ops wrote them."""

    def __init__(self, param_names: Mapping[int, str] | None = None) -> None:
        super().__init__()
        self.param_names: dict[int, str] = dict(param_names or {})
        self.records: list[MatmulRecord] = []
        self.glue_outer: list[MatmulRecord] = []
        self.copies: list[CopyRecord] = []
        self._phase: str | None = None
        self._calls = 0
        self._producers: dict[int, tuple[int, StorageWeakRef]] = {}
        self._by_index: dict[int, MatmulRecord] = {}
        self._param_copies: dict[int, str] = {}
        self._held: list[torch.Tensor] = []

    @contextlib.contextmanager
    def phase(self, name: str) -> Iterator[None]:
        if name not in PHASES:
            raise PhaseError(f"phase must be one of {PHASES}, got {name!r}")
        if self._phase is not None:
            raise PhaseError(f"phase {name!r} entered inside phase {self._phase!r}")
        self._phase = name
        try:
            yield
        finally:
            self._phase = None

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        name = func.overloadpacket.__name__
        ns = func.namespace
        if self._phase is not None and ns not in TRUSTED_NAMESPACES and \
                f"{ns}::{name}" not in ALLOWED_NAMESPACE_OPS:
            raise UnsupportedMatmulError(
                f"{func} reached dispatch inside phase {self._phase!r}: an op outside aten and "
                f"prims may hide a product the capture cannot record")
        if ns == "aten" and name in _FORMS:
            if func._overloadname != "default":
                raise UnsupportedMatmulError(f"{func}: only the .default overload of {name} "
                                             f"is recorded")
            if self._phase is None:
                raise PhaseError(f"{func} ran outside a phase('forward'|'backward') block")
            parsed = self._operands(func, name, args, kwargs)
            out = func(*args, **kwargs)
            self._record(func, name, parsed, out)
            return out
        if func is _TO_COPY and self._phase is not None:
            out = func(*args, **kwargs)
            self._record_copy(args[0], out)
            return out
        if ns == "aten" and name in REJECTED_OPS:
            raise UnsupportedMatmulError(
                f"{func} reached dispatch: the capture records only mm, bmm, addmm and "
                f"baddbmm, so this product would go unchecked (for attention, run the model's "
                f"eager attention)")
        return func(*args, **kwargs)

    @staticmethod
    def _operands(func, name, args, kwargs):
        """``(a, b, bias, alpha, beta)``; a bias outside the bias rule raises."""
        _, has_bias = _FORMS[name]
        if not has_bias:
            return args[0], args[1], None, 1, 1
        bias, a, b = args[0], args[1], args[2]
        beta, alpha = kwargs.get("beta", 1), kwargs.get("alpha", 1)
        vector_once = name == "addmm" and beta == 1 and tuple(bias.shape) == (b.shape[1],)
        # The vector form first: testing a device bias for zeros synchronizes the host.
        if alpha != 1 or not (vector_once or beta == 0 or not bool(bias.ne(0).any())):
            raise BiasedMatmulError(
                f"{func} with beta={beta}, alpha={alpha} and a non-zero bias of shape "
                f"{tuple(bias.shape)}: only a bias vector added once to a non-batched product "
                f"is covered")
        return a, b, bias, alpha, beta

    def _info(self, t: torch.Tensor) -> OperandInfo:
        st = t.untyped_storage()
        ptr = st.data_ptr()
        producer = self._producers.get(ptr)
        if producer is not None and producer[1] != StorageWeakRef(st):
            producer = None
        return OperandInfo(ptr, t.storage_offset(), tuple(t.shape), tuple(t.stride()), t.dtype,
                           self.param_names.get(ptr), None if producer is None else producer[0],
                           self._param_copies.get(ptr))

    def _record_copy(self, src: torch.Tensor, out: torch.Tensor) -> None:
        rec = CopyRecord(len(self.copies), self._phase, self._info(src), self._info(out),
                         StorageWeakRef(out.untyped_storage()))
        if rec.param is not None:
            self._param_copies[rec.out_info.storage_ptr] = rec.param
            self._held.append(out)
        self.copies.append(rec)

    def _record(self, func, name, parsed, out: torch.Tensor) -> None:
        batched, _ = _FORMS[name]
        a, b, bias, alpha, beta = parsed
        rec = MatmulRecord(index=self._calls, op=str(func), phase=self._phase, a=a, b=b,
                           out=out, q=a.shape[-1], batch=a.shape[0] if batched else None,
                           a_info=self._info(a), b_info=self._info(b), out_info=self._info(out),
                           bias=bias, alpha=float(alpha), beta=float(beta),
                           out_storage=StorageWeakRef(out.untyped_storage()))
        rec.versions = {k: t._version for k, t in rec.tensors().items()}
        self._producers[rec.out_info.storage_ptr] = (rec.index, rec.out_storage)
        self._by_index[rec.index] = rec
        self._calls += 1
        (self.glue_outer if rec.q == 1 else self.records).append(rec)

    # ---- after capture -------------------------------------------------------------------

    def wait_copies(self, *, check: bool = True) -> None:
        """The reference waits here for its device-to-host copies; products stay in device
        memory here, so there is nothing to wait for."""

    def release_operands(self) -> None:
        """Drop ``a``, ``b`` and ``bias`` (glue outputs can then be freed), keeping ``out`` and
        the infos."""
        for rec in self.records + self.glue_outer:
            rec.a = rec.b = rec.bias = None
            rec.versions = {k: v for k, v in rec.versions.items() if k == "out"}
        self._held, self._param_copies = [], {}

    def assert_unmodified(self) -> None:
        """Raise :class:`MutatedCaptureError` if a held captured tensor was written in place
        since its capture (invariant 6)."""
        bad = []
        for rec in self.records + self.glue_outer:
            now = {k: t._version for k, t in rec.tensors().items()}
            moved = [k for k, v in rec.versions.items() if now.get(k, v) != v]
            if moved:
                bad.append(f"#{rec.index} {rec.op} ({rec.phase}): {', '.join(moved)}")
        if bad:
            more = f" (+{len(bad) - 10} more)" if len(bad) > 10 else ""
            raise MutatedCaptureError("captured tensors mutated in place after capture: "
                                      + "; ".join(bad[:10]) + more)

    def param_of(self, t: torch.Tensor) -> str | None:
        """The parameter ``t`` aliases, directly or as a copy (until ``release_operands``)."""
        ptr = t.untyped_storage().data_ptr()
        return self.param_names.get(ptr) or self._param_copies.get(ptr)

    @staticmethod
    def is_output_of(t: torch.Tensor, rec: MatmulRecord) -> bool:
        """Whether ``t`` shares the storage of ``rec``'s output (such as the ``W.grad``
        AccumulateGrad adopts); storages compare by identity."""
        return rec.out_storage is not None and \
            rec.out_storage == StorageWeakRef(t.untyped_storage())

    def is_copy_of(self, t: torch.Tensor, index: int) -> bool:
        """Whether ``t`` is a copy of record ``index``'s whole output (such as the fp32 copy
        of a bf16 weight gradient adopted as ``W.grad``)."""
        rec = self._by_index.get(index)
        if rec is None:
            return False
        o = rec.out_info
        whole = (o.storage_offset, o.shape, o.stride)
        mine = StorageWeakRef(t.untyped_storage())
        view = (t.storage_offset(), tuple(t.shape), tuple(t.stride()), t.dtype)
        return any(c.src_info.producer_index == index
                   and (c.src_info.storage_offset, c.src_info.shape, c.src_info.stride) == whole
                   and c.storage == mine
                   and (c.out_info.storage_offset, c.out_info.shape, c.out_info.stride,
                        c.out_info.dtype) == view
                   for c in self.copies)

    @property
    def n_products(self) -> int:
        return sum(r.n_members for r in self.records)

    def summary(self) -> dict:
        ops = Counter((r.phase, r.op) for r in self.records)
        by_phase: Counter[str] = Counter()
        for r in self.records:
            by_phase[r.phase] += r.n_members
        qs = [r.q for r in self.records]
        return {
            "n_calls": len(self.records),
            "n_products": self.n_products,
            "products_by_phase": dict(by_phase),
            "calls_by_phase_op": {f"{p} {o}": n for (p, o), n in sorted(ops.items())},
            "n_glue_outer_calls": len(self.glue_outer),
            "n_glue_outer_products": sum(r.n_members for r in self.glue_outer),
            "n_copies": len(self.copies),
            "n_param_copies": sum(c.param is not None for c in self.copies),
            "q_min": min(qs) if qs else None,
            "q_max": max(qs) if qs else None,
            "output_bytes": sum(r.out.numel() * r.out.element_size() for r in self.records),
            "device_resident": all(r.out.device.type != "cpu" for r in self.records),
        }
