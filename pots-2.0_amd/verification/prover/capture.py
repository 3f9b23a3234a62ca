"""The matmul capture: every matrix product of a training step's forward and backward pass,
recorded with its operands while the products stay in HBM (behaviour of the reference's
verification/prover/capture.py:352-602, ``MatmulCapture``).

The prover runs its step under it, and the verifier's decoder replay runs one pass under it to
learn which call fills which product slot. Usage:

    cap = MatmulCapture(param_names=param_storage_map(model))
    with cap:
        with cap.phase("forward"):
            loss = loss_fn(model(x), y)
        with cap.phase("backward"):
            loss.backward()
    cap.assert_unmodified()

**The recording rules** (a contract: they fix which products a step commits):

- ``aten.mm`` and ``aten.bmm`` (``.default``) each give one :class:`MatmulRecord`; every
  member ``A[i]·B[i]`` of a ``bmm`` is a product of its own.
- ``aten.addmm`` and ``aten.baddbmm`` (``.default``) with ``alpha == 1`` are recorded when
  their added term is inert (``beta == 0``, or a tensor of zeros), and an ``addmm`` also when
  it adds one vector of length ``B.shape[1]`` with ``beta == 1`` (kept as ``bias``). Any other
  added term raises :class:`BiasedMatmulError`.
- A product whose contracted length ``q`` is 1 is an outer product, which is glue: it goes to
  :attr:`MatmulCapture.glue_outer`, not to :attr:`MatmulCapture.records`.
- A matmul-like op of :data:`REJECTED_OPS`, another overload of a handled op, or (inside a
  phase) an op outside the ``aten``/``prims`` namespaces not listed in
  :data:`ALLOWED_NAMESPACE_OPS` raises :class:`UnsupportedMatmulError`; a handled op outside a
  phase raises :class:`PhaseError`.
- ``aten._to_copy`` inside a phase is noted as a :class:`CopyRecord`. A copy of a parameter
  (autocast's bf16 weight, say) is kept alive until :meth:`MatmulCapture.release_operands`,
  and operands that alias it name the parameter in :attr:`OperandInfo.param_copy`. A copy of
  a record's whole output (autocast's fp32 ``W.grad`` of a bf16 weight-gradient product) is
  known through :meth:`MatmulCapture.output_copied_by`. Copies are held only through weak
  references to their storages, so no activation outlives the pass because of the capture.

**How it is built.** Ops are classified once per overload (:func:`_classify`, cached), and the
dispatch hook looks the verdict up and calls its handler. What the capture knows about a
storage (the record whose output it is, or the parameter it copies) lives in one ledger keyed
by the storage's address and checked against a weak reference to the storage itself, since the
allocator may hand a freed address to a new storage. Every tensor the capture holds is
watched: its version counter at capture time is kept, and :meth:`assert_unmodified` reports
any that moved (in-place writes that bypass autograd's counters are not seen).

**Where the products live.** The reference copies each output to pinned host memory as the op
returns and hashes the transcript there. Here a record's ``out`` is the op's own output, on
the device that made it: a C4-shaped step's 50 GB of products fit in one MI355X's 288 GB, and
the leaf hasher reads them where they lie, so the step makes no device-to-host copy at all.
"""

from __future__ import annotations

import contextlib
import enum
import functools
from collections.abc import Callable, Iterator, Mapping
from dataclasses import dataclass, field
from typing import Any

import torch
from torch.multiprocessing.reductions import StorageWeakRef
from torch.utils._python_dispatch import TorchDispatchMode

from verification.computation.matmul_ops import (ALLOWED_NAMESPACE_OPS, HANDLED_OPS,
                                                 REJECTED_OPS, TRUSTED_NAMESPACES)

__all__ = ["PHASES", "CaptureError", "UnsupportedMatmulError", "BiasedMatmulError",
           "PhaseError", "MutatedCaptureError", "OperandInfo", "MatmulRecord", "CopyRecord",
           "MatmulCapture"]

PHASES = ("forward", "backward")


class CaptureError(RuntimeError):
    """The step cannot be captured the way the declared computation needs it."""


class UnsupportedMatmulError(CaptureError):
    """A matrix product reached dispatch in a form the capture does not record."""


class BiasedMatmulError(CaptureError):
    """An addmm/baddbmm whose added term the bias rule does not cover."""


class PhaseError(CaptureError):
    """A product ran outside a phase, or phases were nested."""


class MutatedCaptureError(CaptureError):
    """A captured tensor was written in place after it was captured."""


# ---- what an op is ---------------------------------------------------------------------------

@dataclass(frozen=True)
class _Form:
    """A handled product op: whether it is batched and whether it adds a term."""

    batched: bool
    adds_term: bool


_FORMS: dict[str, _Form] = {
    "mm": _Form(batched=False, adds_term=False),
    "bmm": _Form(batched=True, adds_term=False),
    "addmm": _Form(batched=False, adds_term=True),
    "baddbmm": _Form(batched=True, adds_term=True),
}
if frozenset(_FORMS) != HANDLED_OPS:
    raise ImportError("the capture's product forms differ from HANDLED_OPS")


class _Kind(enum.Enum):
    PRODUCT = enum.auto()        # a handled op's .default overload: record it
    OTHER_OVERLOAD = enum.auto()  # a handled op's other overload (.out, ...): refuse it
    COPY = enum.auto()           # aten._to_copy: note it inside a phase
    REFUSED = enum.auto()        # a matmul-like aten op the inventory cannot hold
    FOREIGN = enum.auto()        # outside the trusted namespaces and the allow list
    PLAIN = enum.auto()          # anything else: run it


@functools.lru_cache(maxsize=None)
def _classify(func: torch._ops.OpOverload) -> tuple[_Kind, _Form | None]:
    """The capture's verdict on one op overload; it depends on the op alone, so it is cached."""
    ns, name = func.namespace, func.overloadpacket.__name__
    if ns == "aten":
        form = _FORMS.get(name)
        if form is not None:
            return (_Kind.PRODUCT if func._overloadname == "default"
                    else _Kind.OTHER_OVERLOAD), form
        if name == "_to_copy" and func._overloadname == "default":
            return _Kind.COPY, None
        if name in REJECTED_OPS:
            return _Kind.REFUSED, None
        return _Kind.PLAIN, None
    if ns in TRUSTED_NAMESPACES or f"{ns}::{name}" in ALLOWED_NAMESPACE_OPS:
        return _Kind.PLAIN, None
    return _Kind.FOREIGN, None


def _term_is_covered(name: str, term: torch.Tensor, b: torch.Tensor, alpha: Any,
                     beta: Any) -> bool:
    """The bias rule for an added term: ``alpha`` must be 1, and the term either one vector of
    B's width added once to a plain product, or inert."""
    if alpha != 1:
        return False
    if name == "addmm" and beta == 1 and tuple(term.shape) == (b.shape[1],):
        return True          # decided on shapes alone, before any look at device values
    return beta == 0 or not bool(term.ne(0).any())


# ---- what a tensor is ------------------------------------------------------------------------

@dataclass(frozen=True)
class OperandInfo:
    """How a captured tensor relates to the pass, for labeling. ``storage_ptr`` identifies the
    storage while the capture holds the tensor. ``producer_index`` is the index of the earlier
    record whose output storage it aliases (``None`` for glue and parameters) and outlives
    :meth:`MatmulCapture.release_operands`. ``param_name`` names the parameter it is a view of,
    ``param_copy`` the parameter it is a ``_to_copy`` of."""

    storage_ptr: int
    storage_offset: int
    shape: tuple[int, ...]
    stride: tuple[int, ...]
    dtype: torch.dtype
    param_name: str | None
    producer_index: int | None = None
    param_copy: str | None = None


@dataclass
class _Origin:
    storage: StorageWeakRef
    producer: int | None = None       # the record whose output this storage is
    copy_of: str | None = None        # the parameter this storage is a copy of
    copy_of_output: int | None = None  # the record whose whole output this storage copies


class _Ledger:
    """Storage address → what made that storage (a record's output, or a copy of a
    parameter); an entry counts only while its weak reference still names the same storage."""

    def __init__(self, params: Mapping[int, str]) -> None:
        self.params = dict(params)
        self._origins: dict[int, _Origin] = {}

    def _origin(self, storage: torch.UntypedStorage) -> _Origin | None:
        o = self._origins.get(storage.data_ptr())
        return o if o is not None and o.storage == StorageWeakRef(storage) else None

    def describe(self, t: torch.Tensor) -> OperandInfo:
        st = t.untyped_storage()
        o = self._origin(st)
        return OperandInfo(storage_ptr=st.data_ptr(), storage_offset=t.storage_offset(),
                           shape=tuple(t.shape), stride=tuple(t.stride()), dtype=t.dtype,
                           param_name=self.params.get(st.data_ptr()),
                           producer_index=None if o is None else o.producer,
                           param_copy=None if o is None else o.copy_of)

    def made_by(self, out: torch.Tensor, index: int) -> StorageWeakRef:
        st = out.untyped_storage()
        ref = StorageWeakRef(st)
        self._origins[st.data_ptr()] = _Origin(ref, producer=index)
        return ref

    def copies_param(self, out: torch.Tensor, param: str) -> None:
        st = out.untyped_storage()
        self._origins[st.data_ptr()] = _Origin(StorageWeakRef(st), copy_of=param)

    def copies_output(self, out: torch.Tensor, index: int) -> None:
        st = out.untyped_storage()
        self._origins[st.data_ptr()] = _Origin(StorageWeakRef(st), copy_of_output=index)

    def produced_by(self, t: torch.Tensor) -> int | None:
        """The index of the record whose output storage ``t`` views, else None."""
        return self._ledger.describe(t).producer_index

    def output_copied_by(self, t: torch.Tensor) -> int | None:
        o = self._origin(t.untyped_storage())
        return None if o is None else o.copy_of_output

    def param_of(self, t: torch.Tensor) -> str | None:
        st = t.untyped_storage()
        named = self.params.get(st.data_ptr())
        if named is not None:
            return named
        o = self._origin(st)
        return None if o is None else o.copy_of

    def drop_param_copies(self) -> None:
        self._origins = {p: o for p, o in self._origins.items() if o.copy_of is None}


# ---- what was recorded -----------------------------------------------------------------------

@dataclass
class MatmulRecord:
    """One captured product call. ``a``, ``b`` and ``bias`` are the tensors the op received
    (``None`` after :meth:`MatmulCapture.release_operands`); ``out`` is its result, in the
    device memory where the op wrote it."""

    index: int          # position among every product-form call of the pass, glue included
    op: str             # "aten.mm.default", ...
    phase: str
    a: torch.Tensor | None
    b: torch.Tensor | None
    out: torch.Tensor
    q: int              # contracted length
    batch: int | None   # members of a bmm/baddbmm, None for a plain product
    a_info: OperandInfo
    b_info: OperandInfo
    out_info: OperandInfo
    bias: torch.Tensor | None = None
    alpha: float = 1.0
    beta: float = 1.0
    out_storage: StorageWeakRef | None = field(default=None, repr=False, compare=False)

    @property
    def n_members(self) -> int:
        return 1 if self.batch is None else self.batch

    def members(self) -> Iterator[tuple[torch.Tensor, torch.Tensor, torch.Tensor]]:
        """``(A_i, B_i, P_i)`` for each checked product of the call."""
        if self.a is None or self.b is None:
            raise CaptureError(f"record #{self.index}: operands were released")
        if self.batch is None:
            yield self.a, self.b, self.out
        else:
            yield from zip(self.a.unbind(0), self.b.unbind(0), self.out.unbind(0))


@dataclass
class CopyRecord:
    """One ``aten._to_copy`` inside a phase. ``storage`` refers to the copy's storage weakly
    (its identity only)."""

    index: int
    phase: str
    src_info: OperandInfo
    out_info: OperandInfo
    storage: StorageWeakRef = field(repr=False)

    @property
    def param(self) -> str | None:
        """The parameter this copies, directly or through an earlier copy of it."""
        return self.src_info.param_name or self.src_info.param_copy


@dataclass
class _Watched:
    record: MatmulRecord
    role: str           # "a", "b", "out" or "bias"
    version: int


# ---- the capture -----------------------------------------------------------------------------

class MatmulCapture(TorchDispatchMode):
    """A passthrough dispatch mode that records every product of a forward and backward
    pass, the products staying where the ops wrote them."""

    def __init__(self, param_names: Mapping[int, str] | None = None) -> None:
        super().__init__()
        self.records: list[MatmulRecord] = []
        self.glue_outer: list[MatmulRecord] = []
        self.copies: list[CopyRecord] = []
        self._ledger = _Ledger(param_names or {})
        self._watched: list[_Watched] = []
        self._param_copy_tensors: list[torch.Tensor] = []  # kept alive until release
        self._current: str | None = None
        self._calls = 0
        self._made: dict[int, MatmulRecord] = {}  # record index -> record, glue included
        self._handlers: dict[_Kind, Callable[..., Any]] = {
            _Kind.PRODUCT: self._on_product,
            _Kind.OTHER_OVERLOAD: self._on_other_overload,
            _Kind.COPY: self._on_copy,
            _Kind.REFUSED: self._on_refused,
            _Kind.FOREIGN: self._on_foreign,
            _Kind.PLAIN: self._on_plain,
        }

    @property
    def param_names(self) -> dict[int, str]:
        return self._ledger.params

    @contextlib.contextmanager
    def phase(self, name: str) -> Iterator[None]:
        """Products run inside exactly one phase, forward or backward."""
        if name not in PHASES:
            raise PhaseError(f"phase must be one of {PHASES}, got {name!r}")
        if self._current is not None:
            raise PhaseError(f"phase {name!r} entered inside phase {self._current!r}")
        self._current = name
        try:
            yield
        finally:
            self._current = None

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        kind, form = _classify(func)
        return self._handlers[kind](func, form, args, kwargs or {})

    # -- handlers, one per verdict of _classify

    def _on_plain(self, func, form, args, kwargs):
        return func(*args, **kwargs)

    def _on_foreign(self, func, form, args, kwargs):
        if self._current is not None:
            raise UnsupportedMatmulError(
                f"{func} reached dispatch inside phase {self._current!r}: an op outside aten "
                f"and prims may hide a product the capture cannot record")
        return func(*args, **kwargs)

    def _on_refused(self, func, form, args, kwargs):
        raise UnsupportedMatmulError(
            f"{func} reached dispatch: the capture records only mm, bmm, addmm and baddbmm, "
            f"so this product would go unchecked (for attention, run the model's eager "
            f"attention)")

    def _on_other_overload(self, func, form, args, kwargs):
        raise UnsupportedMatmulError(f"{func}: only the .default overload of "
                                     f"{func.overloadpacket.__name__} is recorded")

    def _on_copy(self, func, form, args, kwargs):
        out = func(*args, **kwargs)
        if self._current is not None:
            src = args[0] if args else kwargs["self"]
            note = CopyRecord(len(self.copies), self._current, self._ledger.describe(src),
                              self._ledger.describe(out), StorageWeakRef(out.untyped_storage()))
            if note.param is not None:
                self._ledger.copies_param(out, note.param)
                self._param_copy_tensors.append(out)
            elif note.src_info.producer_index is not None:
                made = self._made[note.src_info.producer_index]
                if src.numel() == made.out.numel() and \
                        src.storage_offset() == made.out.storage_offset():
                    self._ledger.copies_output(out, made.index)
            self.copies.append(note)
        return out

    def _on_product(self, func, form: _Form, args, kwargs):
        if self._current is None:
            raise PhaseError(f"{func} ran outside a phase('forward'|'backward') block")
        name = func.overloadpacket.__name__
        if form.adds_term:
            term, a, b = args[0], args[1], args[2]
            alpha, beta = kwargs.get("alpha", 1), kwargs.get("beta", 1)
            if not _term_is_covered(name, term, b, alpha, beta):
                raise BiasedMatmulError(
                    f"{func} with beta={beta}, alpha={alpha} and a non-zero bias of shape "
                    f"{tuple(term.shape)}: only a bias vector added once to a non-batched "
                    f"product is covered")
        else:
            term, (a, b), alpha, beta = None, args[:2], 1, 1
        out = func(*args, **kwargs)
        index = self._calls
        self._calls += 1
        d = self._ledger.describe
        rec = MatmulRecord(index=index, op=str(func), phase=self._current, a=a, b=b, out=out,
                           q=int(a.shape[-1]), batch=int(a.shape[0]) if form.batched else None,
                           a_info=d(a), b_info=d(b), out_info=d(out), bias=term,
                           alpha=float(alpha), beta=float(beta))
        rec.out_storage = self._ledger.made_by(out, index)
        self._made[index] = rec
        for role in ("a", "b", "out", "bias"):
            t = getattr(rec, role)
            if t is not None:
                self._watched.append(_Watched(rec, role, t._version))
        (self.records if rec.q != 1 else self.glue_outer).append(rec)
        return out

    # ---- after the pass ------------------------------------------------------------------

    def release_operands(self) -> None:
        """Let go of every record's ``a``, ``b`` and ``bias`` (so glue can be freed) and of the
        parameter copies; ``out`` and the infos stay."""
        for rec in (*self.records, *self.glue_outer):
            rec.a = rec.b = rec.bias = None
        self._watched = [w for w in self._watched if w.role == "out"]
        self._param_copy_tensors = []
        self._ledger.drop_param_copies()

    def assert_unmodified(self) -> None:
        """Raise :class:`MutatedCaptureError` when a tensor the capture still holds was
        written in place after its capture."""
        moved: dict[int, list[str]] = {}
        for w in self._watched:
            t = getattr(w.record, w.role)
            if t is not None and t._version != w.version:
                moved.setdefault(w.record.index, []).append(w.role)
        if not moved:
            return
        by_index = {r.index: r for r in (*self.records, *self.glue_outer)}
        lines = [f"#{i} {by_index[i].op} ({by_index[i].phase}): {', '.join(roles)}"
                 for i, roles in sorted(moved.items())]
        tail = f" (+{len(lines) - 10} more)" if len(lines) > 10 else ""
        raise MutatedCaptureError("captured tensors mutated in place after capture: "
                                  + "; ".join(lines[:10]) + tail)

    def param_of(self, t: torch.Tensor) -> str | None:
        """The parameter ``t`` views or copies (copies are known until release)."""
        return self._ledger.param_of(t)

    @staticmethod
    def is_output_of(t: torch.Tensor, rec: MatmulRecord) -> bool:
        """Whether ``t``'s storage is ``rec``'s output storage (as when AccumulateGrad adopts
        a weight gradient's product as ``W.grad``); storages compare by identity."""
        return rec.out_storage is not None and \
            rec.out_storage == StorageWeakRef(t.untyped_storage())

    def produced_by(self, t: torch.Tensor) -> int | None:
        """The index of the record whose output storage ``t`` views, else None."""
        return self._ledger.describe(t).producer_index

    def output_copied_by(self, t: torch.Tensor) -> int | None:
        """The index of the record whose whole output ``t``'s storage is a ``_to_copy`` of
        (as autocast's fp32 ``W.grad`` copies a bf16 weight-gradient product), else None."""
        return self._ledger.output_copied_by(t)

    @property
    def n_products(self) -> int:
        return sum(r.n_members for r in self.records)

    def summary(self) -> dict[str, Any]:
        """Counts for the step's report: product calls and checked products, per phase and
        per op; the q = 1 glue calls; copies and parameter copies; the range of contracted
        lengths; the products' bytes and whether they all stayed on the device."""
        per_phase = dict.fromkeys(PHASES, 0)
        per_op: dict[str, int] = {}
        nbytes, on_device = 0, True
        for r in self.records:
            per_phase[r.phase] += r.n_members
            per_op[f"{r.phase}:{r.op}"] = per_op.get(f"{r.phase}:{r.op}", 0) + 1
            nbytes += r.out.numel() * r.out.element_size()
            on_device = on_device and r.out.device.type != "cpu"
        qs = [r.q for r in self.records]
        return {
            "calls": len(self.records),
            "products": self.n_products,
            "products_per_phase": {p: n for p, n in per_phase.items() if n},
            "calls_per_op": per_op,
            "outer_calls": len(self.glue_outer),
            "outer_products": sum(r.n_members for r in self.glue_outer),
            "copies": len(self.copies),
            "parameter_copies": sum(1 for c in self.copies if c.param is not None),
            "q_range": (min(qs), max(qs)) if qs else None,
            "product_bytes": nbytes,
            "on_device": on_device,
        }
