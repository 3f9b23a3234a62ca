"""The declared computation ``C``: the transcript layout and the product inventory.

Reference: verification/computation/interface.py:60-330. Only the layout contract the hot
path needs is kept: ``ProductSpec`` (which leaf is ``P_m``, its shapes, its challenge width),
the leaf order ``[records n_s | W_t n_w | P_1..P_M | W_{t+1} n_w]``, the index helpers, and
check 6a's declaration (the step size ``eta``, ``linear_weights``, ``chain_gradient``).
A computation serves check 5's operands through :meth:`DeclaredComputation.replay`: the
decoder takes the captured operands it is given (its model replay is not part of this build),
the MLP instance replays its glue from the committed leaves. The prover's side
(:meth:`~DeclaredComputation.build_model`, :meth:`~DeclaredComputation.loss`,
:meth:`~DeclaredComputation.forward_backward`, :meth:`~DeclaredComputation.label`;
reference interface.py:362-413) drives ``verification.prover.step.prove_step``.
"""

from __future__ import annotations

import abc
import contextlib
import enum
from collections.abc import Callable, Iterable, Mapping, Sequence
from dataclasses import dataclass
from functools import cached_property
from typing import Any

import torch

HOST = torch.device("cpu")


class ProductKind(enum.Enum):
    FORWARD = "forward"
    WEIGHT_GRAD = "weight_grad"
    INPUT_GRAD = "input_grad"
    OPERAND_GRAD = "operand_grad"


@dataclass(frozen=True)
class ProductSpec:
    """One product ``P_m = A·B`` of the inventory.

    ``member`` is the ``(s, h)`` index of one member of a batched attention product, or
    ``None``. ``bias`` names the declared weight ``b`` the same op adds (``P = A·B + 1·bᵀ``);
    check 5 then checks ``[A | 1]·[B ; bᵀ]`` and ``q`` is one greater.
    """

    m: int
    name: str
    kind: ProductKind
    a_shape: tuple[int, int]
    b_shape: tuple[int, int]
    weight: str | None = None
    layer: int | None = None
    member: tuple[int, ...] | None = None
    bias: str | None = None

    def __post_init__(self) -> None:
        if self.m < 1:
            raise ValueError(f"{self.name}: m must be 1-based, got {self.m}")
        if len(self.a_shape) != 2 or len(self.b_shape) != 2:
            raise ValueError(f"{self.name}: operands must be matrices")
        if self.a_shape[1] != self.b_shape[0]:
            raise ValueError(f"{self.name}: A {self.a_shape} and B {self.b_shape} don't chain")

    @property
    def p_shape(self) -> tuple[int, int]:
        return (self.a_shape[0], self.b_shape[1])

    @property
    def q(self) -> int:
        """Contracted length of the checked matmul (one more with a bias)."""
        return self.a_shape[1] + (self.bias is not None)

    @property
    def width(self) -> int:
        """Challenge length: the column count of ``P``."""
        return self.b_shape[1]


class Replay(abc.ABC):
    """The operands of each product, as the verifier serves them to check 5."""

    @abc.abstractmethod
    def operands(self, m: int) -> tuple[torch.Tensor, torch.Tensor]:
        """``(A_m, B_m)`` of product ``m``."""

    def operand_group(self, ms: Sequence[int],
                      dtype: torch.dtype | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """The operands of products ``ms`` (one shape pair) stacked ``[len(ms), ·, ·]``, equal
        to ``torch.stack`` of ``operands(m)`` over ``ms`` (reference interface.py:143-162).
        Without ``dtype`` an instance may return views of tensors it holds (a batched
        product's whole operands) instead of copies; the caller must not write to them. This
        default stacks member by member. An error is the first one ``operands`` raises."""
        pairs = [self.operands(m) for m in ms]
        a = torch.stack([p[0] for p in pairs])
        b = torch.stack([p[1] for p in pairs])
        if dtype is not None:
            a, b = a.to(dtype), b.to(dtype)
        return a, b


class LabelingError(RuntimeError):
    """Captured matmuls do not map one to one onto the declared product slots."""


def load_weights(computation: DeclaredComputation, model: torch.nn.Module,
                 weights: Mapping[str, torch.Tensor]) -> None:
    """Copy ``weights`` into ``model``; both hold exactly the declared weights (reference
    interface.py:183-198)."""
    params = dict(model.named_parameters())
    names = set(computation.weight_names)
    if set(params) != names:
        raise ValueError(f"model parameters {sorted(params)} differ from the declared weights")
    if set(weights) != names:
        raise ValueError(f"weights {sorted(weights)} differ from the declared weights")
    with torch.no_grad():
        for name in computation.weight_names:
            w, p = weights[name], params[name]
            if w.shape != p.shape or w.dtype != p.dtype:
                raise ValueError(f"{name}: got {w.dtype} {tuple(w.shape)}, the model holds "
                                 f"{p.dtype} {tuple(p.shape)}")
            p.copy_(w)


def snapshot_weights(computation: DeclaredComputation,
                     model: torch.nn.Module) -> dict[str, torch.Tensor]:
    """Copies of the model's declared weights, in ``weight_names`` order, on the device the
    model is on (reference interface.py:201-212 copies them to the host; here a step's
    ``W_{t+1}`` leaves stay in HBM for the device commit)."""
    return {n: model.get_parameter(n).detach().clone() for n in computation.weight_names}


def chain_gradient(parts: Iterable[torch.Tensor], dtype: torch.dtype) -> torch.Tensor:
    """A weight's gradient from its committed weight-gradient products: each widened to
    ``dtype`` and added in order, out of place, ``((P_0 + P_1) + P_2) + …`` (reference
    interface.py:169-180). One part is that part widened."""
    g: torch.Tensor | None = None
    for p in parts:
        g = p.to(dtype) if g is None else g + p.to(dtype)
    if g is None:
        raise ValueError("a gradient needs at least one product")
    return g


class DeclaredComputation(abc.ABC):
    """The layout and inventory of one step's transcript."""

    @property
    @abc.abstractmethod
    def n_s(self) -> int:
        """Records (sequences) per step."""

    @property
    @abc.abstractmethod
    def weight_names(self) -> tuple[str, ...]:
        ...

    @property
    @abc.abstractmethod
    def weight_shapes(self) -> dict[str, tuple[int, ...]]:
        ...

    @property
    @abc.abstractmethod
    def products(self) -> tuple[ProductSpec, ...]:
        ...

    @property
    def eta(self) -> float:
        """The constant SGD step size, fixed in ``C`` (reference interface.py:225-228)."""
        raise NotImplementedError(f"{type(self).__name__} declares no step size")

    @property
    def linear_weights(self) -> dict[str, tuple[int, ...]]:
        """Check 6a: weight name -> the ``m`` of the committed weight-gradient products whose
        :func:`chain_gradient`, in this order, is its whole gradient (reference
        interface.py:245-249). None by default."""
        return {}

    @property
    def glue_gradient_weights(self) -> tuple[str, ...]:
        """Check 6b's weights: those whose gradient is (or includes) glue the replay
        recomputes, every weight that is not linear, in leaf order (reference
        interface.py:288-290)."""
        return tuple(n for n in self.weight_names if n not in self.linear_weights)

    @property
    def weight_dtype(self) -> torch.dtype:
        return torch.float32

    @property
    def product_dtype(self) -> torch.dtype:
        return torch.float32

    @property
    def operand_dtype(self) -> torch.dtype:
        return self.product_dtype

    @property
    def accumulator_dtype(self) -> torch.dtype:
        """The matmuls accumulate in fp32 (reference interface.py:269)."""
        return torch.float32

    def replay(self, leaves: Any) -> Replay:
        """Check 5's operands for the committed ``leaves`` (reference interface.py:380).

        By default a computation serves operands it was given with :meth:`use_operands` (the
        exact operands the prover used, as a capture records them); a subclass that replays
        its glue from the leaves (the MLP instance) overrides this method."""
        r = getattr(self, "_operands", None)
        if r is None:
            raise NotImplementedError(
                f"{type(self).__name__} has no operand source: the model replay is not part "
                f"of this build; give the captured operands with use_operands()")
        return r

    def use_operands(self, replay: Replay | None) -> None:
        """Serve ``replay``'s operands to check 5 (``None`` removes them)."""
        self._operands = replay

    def encode_record(self, record: Any) -> bytes:
        from setup.records import encode_record
        return encode_record(record)

    def record_leaf(self, record: Any) -> tuple[int, torch.Tensor] | None:
        """``(tag, tensor)`` when a record's leaf is a tensor leaf (its encoding is
        ``encode_tensor_leaf(tag, tensor)``), so a hasher can read its payload where it lies;
        ``None`` (the default) when only :meth:`encode_record` gives its bytes. Validates the
        record as :meth:`encode_record` does."""
        return None

    # ---- prover side (reference interface.py:362-413; the verifier never calls these) ----

    def build_model(self) -> torch.nn.Module:
        """A fresh model whose parameters are exactly :attr:`weight_names`."""
        raise NotImplementedError(f"{type(self).__name__} builds no model in this build")

    def loss(self, model: torch.nn.Module, records: Sequence[Any]) -> torch.Tensor:
        """Assemble the batch and run the forward pass to the scalar loss."""
        raise NotImplementedError(f"{type(self).__name__} has no training loss in this build")

    def forward_backward(self, model: torch.nn.Module, records: Sequence[Any],
                         stage: Callable[[str], contextlib.AbstractContextManager[Any]]
                         ) -> torch.Tensor:
        """One training pass: the forward pass to the loss inside ``stage("forward")``, then
        ``loss.backward()`` inside ``stage("backward")``; returns the loss."""
        with stage("forward"):
            loss = self.loss(model, records)
        with stage("backward"):
            loss.backward()
        return loss

    def label(self, capture: Any, model: torch.nn.Module) -> list[torch.Tensor]:
        """The captured outputs in canonical order ``P_1..P_M``, mapped by operand identity;
        :class:`LabelingError` unless every slot is filled once with its declared shape."""
        raise NotImplementedError(f"{type(self).__name__} labels no capture in this build")

    def product_class(self, spec: ProductSpec) -> str:
        """The κ class of a product; by default its kind and role with layer digits masked."""
        import re
        role = spec.weight if spec.weight is not None else spec.name
        return f"{spec.kind.value}:{re.sub(r'[0-9]+', '*', role)}"

    @cached_property
    def operand_groups(self) -> tuple[tuple[int, ...], ...]:
        """Product indices (0-based, canonical order) grouped as a step holds their operands:
        the members of one batched attention product (one layer, one role such as ``L2.dA``,
        one operand shape pair) form a group, in canonical order, even where two roles of a
        backward block interleave (``dA[0,0], dV[0,0], dA[0,1], …``); every other product
        is a group of its own. Groups are listed in order of their first product. A replay
        serves a group with one :meth:`Replay.operand_group` call."""
        out: list[list[int]] = []
        at: dict[tuple[Any, ...], int] = {}
        for i, s in enumerate(self.products):
            if s.member is None:
                out.append([i])
                continue
            key = (s.name.split("[", 1)[0], s.kind, s.a_shape, s.b_shape)
            g = at.get(key)
            if g is None:
                at[key] = len(out)
                out.append([i])
            else:
                out[g].append(i)
        return tuple(tuple(g) for g in out)

    @property
    def M(self) -> int:
        return len(self.products)

    @property
    def n_w(self) -> int:
        return len(self.weight_names)

    @property
    def n_leaves(self) -> int:
        return self.n_s + 2 * self.n_w + self.M

    def product(self, m: int) -> ProductSpec:
        if not 1 <= m <= self.M:
            raise IndexError(f"product m={m} outside 1..{self.M}")
        return self.products[m - 1]

    @cached_property
    def _weight_pos(self) -> dict[str, int]:
        return {n: i for i, n in enumerate(self.weight_names)}

    def record_index(self, i: int) -> int:
        if not 0 <= i < self.n_s:
            raise IndexError(f"record {i} outside 0..{self.n_s - 1}")
        return i

    def w_t_index(self, name: str) -> int:
        return self.n_s + self._weight_pos[name]

    def product_index(self, m: int) -> int:
        self.product(m)
        return self.n_s + self.n_w + m - 1

    def w_next_index(self, name: str) -> int:
        return self.n_s + self.n_w + self.M + self._weight_pos[name]

    def validate(self) -> None:
        """Raise ``ValueError`` if the declaration is internally inconsistent."""
        names = self.weight_names
        if len(set(names)) != len(names):
            raise ValueError("duplicate weight names")
        if set(self.weight_shapes) != set(names):
            raise ValueError("weight_shapes keys differ from weight_names")
        for i, p in enumerate(self.products, start=1):
            if p.m != i:
                raise ValueError(f"product {p.name} has m={p.m} at position {i}")
            if p.q < 2:
                raise ValueError(f"product {p.name} has q={p.q}; a q=1 product is glue")
            if p.weight is not None and p.weight not in self._weight_pos:
                raise ValueError(f"product {p.name} names unknown weight {p.weight}")
            if p.bias is not None:
                if p.bias not in self._weight_pos:
                    raise ValueError(f"product {p.name} names unknown bias {p.bias}")
                if p.member is not None:
                    raise ValueError(f"member product {p.name} names a bias")
                if tuple(self.weight_shapes[p.bias]) != (p.width,):
                    raise ValueError(f"bias {p.bias} of {p.name} is not of P's width")
