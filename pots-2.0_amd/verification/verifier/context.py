"""What the per-step checks share: the step context, rejections, statistics and the error guard.

Reference: verification/verifier/context.py (``Rejection`` :82-98, ``ProductStat`` :101-125,
``StepState`` :231-253, ``StepContext`` :256-311, ``CommittedLeaves`` :196-228, ``_guard`` /
``_checked`` :314-338). The names, fields and semantics are the reference's, so callers and
tests written against it work unchanged:

- a check returns ``None`` or a :class:`Rejection` ``(step, check_id, detail, kind)``, with
  ``kind`` ``"malformed"`` when prover data failed to read, decode or validate and
  ``"failed"`` when well-formed data failed the check;
- :class:`StepContext` holds the verifier's own knowledge for one step, and its
  :class:`StepState` what one check derives for a later one (check 2's claimed root, leaf
  hashes and committed leaves; check 2's recomputed root);
- every product check 5 judges is recorded as a :class:`ProductStat`, judged or not;
- :func:`_guard` turns a prover-data error into a ``"malformed"`` rejection at the check
  that read the leaf.
"""

from __future__ import annotations

import functools
import math
from collections.abc import Callable, Iterable, Iterator
from contextlib import AbstractContextManager, contextmanager, nullcontext
from dataclasses import dataclass, field
from typing import TYPE_CHECKING, Any, Literal

import torch

from setup.records import Record
from verification.commitment.merkle import DIGEST_SIZE
from verification.parameters import UNIT_ROUNDOFF
from verification.transcript.errors import LeafShapeError, StoreMutationError, \
    TranscriptFormatError

if TYPE_CHECKING:
    from verification.computation.interface import DeclaredComputation, ProductSpec, Replay
    from verification.verifier.matmul_check.freivalds import ProductMeasure

__all__ = ["PROVER_DATA_ERRORS", "Section", "no_section", "Rejection", "RejectionKind",
           "ProductStat", "TensorStat", "StepStats", "StepState", "StepContext",
           "CommittedLeaves"]

Section = Callable[[str], AbstractContextManager[Any]]
_NO_SECTION = nullcontext()


def no_section(name: str) -> AbstractContextManager[Any]:
    """The metrics seam when nothing is measured: a shared no-op context manager."""
    return _NO_SECTION


# Prover-data errors: TranscriptFormatError and its subclasses, EncodingError, NonFiniteError
# and a record's ValueError all derive from ValueError; a missing index is a LookupError.
PROVER_DATA_ERRORS: tuple[type[BaseException], ...] = (ValueError, LookupError)

RejectionKind = Literal["malformed", "failed"]


@dataclass(frozen=True)
class Rejection:
    """``(step, check_id, detail)``, and whether the data was malformed or failed the check."""

    step: int
    check_id: str
    detail: str
    kind: RejectionKind = "failed"


@dataclass(frozen=True)
class ProductStat:
    """Check 5's numbers for one product: ``κ_m`` and the ``k`` normalized residuals, plus
    the scale (``q``, ``‖P‖_F``, ``ν``, ``‖|P|·1‖``, ``U``), kept out of equality."""

    m: int
    name: str
    cls: str
    kappa: float
    normalized: tuple[float, ...]
    q: int = field(default=0, compare=False)
    p_norm: float = field(default=math.nan, compare=False)
    nu: float = field(default=math.nan, compare=False)
    p_abs1: float = field(default=math.nan, compare=False)
    u: float = field(default=math.nan, compare=False)


@dataclass(frozen=True)
class TensorStat:
    """Check 6's number for one weight: ``ρ_max = max_i |R_i| / (ε_W·(|W_t,i| + |η·G_i|))``
    (reference context.py:128-133)."""

    weight: str
    check_id: str
    rho_max: float


class StepStats:
    """One step's statistics: check 5's per product and check 6's per weight, in the order
    the checks judged them. Check 5 may give its products as columns
    (:meth:`add_products`), made into :class:`ProductStat` records when first read."""

    def __init__(self, products: list[ProductStat] | None = None,
                 tensors: list[TensorStat] | None = None,
                 operands_from_prover: bool = False) -> None:
        self._products: list[ProductStat] = list(products or [])
        self._pending: list[Callable[[], Iterable[ProductStat]]] = []
        self.tensors: list[TensorStat] = list(tensors or [])
        # check 5 measured the prover's captured operands, not a replay of the committed
        # leaves
        self.operands_from_prover = operands_from_prover

    @property
    def products(self) -> list[ProductStat]:
        if self._pending:
            pending, self._pending = self._pending, []
            for make in pending:
                self._products.extend(make())
        return self._products

    def add_products(self, make: Callable[[], Iterable[ProductStat]]) -> None:
        """Products to append after those recorded so far, made by ``make()`` on first
        read."""
        self._pending.append(make)

    def __repr__(self) -> str:
        return (f"StepStats(products={self.products!r}, tensors={self.tensors!r}, "
                f"operands_from_prover={self.operands_from_prover!r})")

    def __eq__(self, other: object) -> bool:
        if not isinstance(other, StepStats):
            return NotImplemented
        return (self.products, self.tensors, self.operands_from_prover) == \
            (other.products, other.tensors, other.operands_from_prover)

    def max_normalized(self) -> float:
        return max((max(p.normalized) for p in self.products), default=0.0)

    def max_kappa(self) -> float:
        return max((p.kappa for p in self.products), default=0.0)

    def by_class(self) -> dict[str, list[ProductStat]]:
        out: dict[str, list[ProductStat]] = {}
        for p in self.products:
            out.setdefault(p.cls, []).append(p)
        return out


def _leaf_tensors(obj: Any) -> list[torch.Tensor]:
    if isinstance(obj, torch.Tensor):
        return [obj]
    if isinstance(obj, Record):
        return [obj.ids, obj.targets, obj.mask]
    raise LeafShapeError(f"unsupported leaf object {type(obj).__name__}")


class CommittedLeaves:
    """The leaves check 2 hashed, served to every later check.

    Each tensor's ``_version`` is recorded when the leaf is added and compared on every read,
    so an in-place write through any alias after hashing raises :class:`StoreMutationError`
    instead of serving changed bytes. A tensor leaf keeps its one version as an int, a record
    the tuple of its tensors' versions.
    """

    def __init__(self) -> None:
        self._objs: list[Any] = []
        self._versions: list[int | tuple[int, ...]] = []

    @staticmethod
    def _version(obj: Any) -> int | tuple[int, ...]:
        if isinstance(obj, torch.Tensor):
            return obj._version
        return tuple(t._version for t in _leaf_tensors(obj))

    def add(self, obj: Any) -> None:
        self._versions.append(self._version(obj))
        self._objs.append(obj)

    @classmethod
    def of(cls, objs: list[Any]) -> CommittedLeaves:
        """The leaves ``objs``, in order, as if added one by one."""
        out = cls()
        version, tensor = cls._version, torch.Tensor
        out._versions = [o._version if type(o) is tensor else version(o) for o in objs]
        out._objs = list(objs)
        return out

    def __len__(self) -> int:
        return len(self._objs)

    def changed(self, index: int) -> bool:
        return self._version(self._objs[index]) != self._versions[index]

    def first_changed(self) -> int | None:
        """The first leaf written in place since it was added, or ``None``."""
        version, tensor = self._version, torch.Tensor
        now = [o._version if type(o) is tensor else version(o) for o in self._objs]
        if now == self._versions:
            return None
        return next(i for i, (a, b) in enumerate(zip(now, self._versions)) if a != b)

    def leaf(self, index: int) -> Any:
        # Indices come from C, never from the prover, so a bad one is a verifier bug.
        if not (isinstance(index, int) and 0 <= index < len(self._objs)):
            raise RuntimeError(f"committed leaf index {index!r} outside 0..{len(self._objs) - 1}")
        obj = self._objs[index]
        if self._version(obj) != self._versions[index]:
            raise StoreMutationError(f"leaf {index} changed in place after check 2 hashed it")
        return obj

    def objects(self) -> list[Any]:
        """Every leaf object, in order, without the version test (for one batched read right
        after hashing, when nothing can have run in between)."""
        return list(self._objs)


@dataclass
class StepState:
    """What a check derives for a later one; empty at step start."""

    early_hashes: dict[int, bytes] = field(default_factory=dict)
    claimed_root: bytes | None = None
    leaf_hashes: list[bytes] | None = None
    recomputed_root: bytes | None = None
    leaves: CommittedLeaves | None = None
    replay: Replay | None = None
    run_rest: list[tuple[ProductSpec, ProductMeasure]] = field(default_factory=list)
    run_rest_error: Exception | None = None

    def committed(self) -> CommittedLeaves:
        if self.leaves is None:
            raise RuntimeError("this check reads check 2's committed leaves; run check 2 first")
        return self.leaves


@dataclass
class StepContext:
    """The verifier's own knowledge for one step. Nothing in it comes from the prover."""

    step: int
    indices: tuple[int, ...]
    h_D: bytes
    n_records: int
    prev_w_hashes: tuple[bytes, ...]
    chain_check_id: str
    k: int
    eps_in: float
    eps_acc: float
    eps_w: float
    judge: bool = True
    kappa_guard: bool = True
    trust_prover_operands: bool = False
    # the verifier's plan cache (verification.verifier.plans.PlanCache), kept across steps
    plans: Any = None
    state: StepState = field(default_factory=StepState)
    stats: StepStats = field(default_factory=StepStats)
    section: Section | None = None

    def timed(self, name: str) -> AbstractContextManager[Any]:
        return _NO_SECTION if self.section is None else self.section(name)

    def hash_stats(self) -> Any:
        from verification.commitment.leaves import HashStats
        return HashStats() if hasattr(self.section, "add") else None

    def stamp(self, name: str, run: int = -1, group: int = -1,
              window: int = -1) -> AbstractContextManager[Any]:
        f = getattr(self.section, "stamp", None)
        return _NO_SECTION if f is None else f(name, run, group, window)

    @classmethod
    def for_computation(cls, c: DeclaredComputation, **kw: Any) -> StepContext:
        """Fill the unit roundoffs from ``C``'s declared dtypes unless given."""
        kw.setdefault("eps_in", UNIT_ROUNDOFF[c.operand_dtype])
        kw.setdefault("eps_acc", UNIT_ROUNDOFF[c.accumulator_dtype])
        kw.setdefault("eps_w", UNIT_ROUNDOFF[c.weight_dtype])
        return cls(**kw)

    def reject(self, check_id: str, detail: str, kind: RejectionKind = "failed") -> Rejection:
        return Rejection(self.step, check_id, detail, kind)


class _Rejected(Exception):
    def __init__(self, rejection: Rejection) -> None:
        self.rejection = rejection


@contextmanager
def _guard(ctx: StepContext, check_id: str,
           errors: tuple[type[BaseException], ...] = PROVER_DATA_ERRORS) -> Iterator[None]:
    """Map a prover-data error raised inside the block to a ``"malformed"`` rejection."""
    try:
        yield
    except errors as e:
        raise _Rejected(ctx.reject(check_id, f"malformed prover data: "
                                             f"{type(e).__name__}: {e}", "malformed")) from e


_AFTER_COMMIT: tuple[type[BaseException], ...] = (TranscriptFormatError,)


def _checked(fn: Callable[..., Rejection | None]) -> Callable[..., Rejection | None]:
    @functools.wraps(fn)
    def run(*args: Any) -> Rejection | None:
        try:
            return fn(*args)
        except _Rejected as r:
            return r.rejection
    return run


def _is_digest(x: Any) -> bool:
    return isinstance(x, bytes) and len(x) == DIGEST_SIZE
