"""The small MLP instance of the declared computation, and its replay on the GPU.

What is kept from the reference (verification/computation/instances/mlp.py:1-365) because a
transcript's leaves depend on it: the model, the record format, the weight names and the
canonical product order.

- **Model.** ``L = len(widths) − 1`` bias-free linears ``Y_ℓ = X_ℓ·W_ℓᵀ``, ``X_{ℓ+1} =
  tanh(Y_ℓ)`` between them, and the mean squared error of ``Y_L`` against the targets.
  ``X_1`` is batch data, so the step has no ``δX_1`` and ``M = 3L − 1``.
- **Record.** A float32 vector ``x ‖ y`` of ``d_in + d_out`` entries; its leaf is the tensor
  leaf with tag ``0x04``.
- **Weights.** ``layers.{ℓ−1}.weight`` of shape ``[o, i]``, ``ℓ = 1..L``, all linear (check
  6a covers each through ``G_ℓ``).
- **Order.** ``Y_1 … Y_L``, then for ``ℓ = L … 1``: ``dX_ℓ`` (``ℓ ≥ 2``) and ``G_ℓ``.

======== ============ ======== ===========
product  A            B        P
======== ============ ======== ===========
Y_ℓ      X_ℓ          W_ℓᵀ     n_s × o
dX_ℓ     δY_ℓ         W_ℓ      n_s × i
G_ℓ      δY_ℓᵀ        X_ℓ      o × i
======== ============ ======== ===========

with ``δY_L = ∂loss/∂Y_L`` and ``δY_ℓ = dX_{ℓ+1} ⊙ tanh′(Y_ℓ)``.

:class:`MLPReplay` is the verifier's glue: every operand from the committed leaves, on the GPU.
``X_{ℓ+1}`` is ``tanh`` of the committed ``Y_ℓ``; ``δY_ℓ`` comes from autograd through the
model's own ``act`` and ``loss_fn`` at the committed ``Y_ℓ`` (and ``dX_{ℓ+1}``). The operands go
to the Freivalds kernels as they are, ``W_ℓᵀ`` and ``δY_ℓᵀ`` as transposed views.
"""

from __future__ import annotations

import math
from collections.abc import Iterator, Sequence
from functools import cached_property
from typing import Any

import torch
from torch import nn

from verification.commitment.encoding import TAG_MLP_RECORD, encode_tensor_leaf
from verification.computation.interface import (DeclaredComputation, LabelingError,
                                               ProductKind, ProductSpec, Replay, load_weights)

__all__ = ["DEFAULT_WIDTHS", "MLP", "MLPComputation", "MLPReplay", "make_record",
           "split_record", "init_weights", "synthetic_dataset"]

DEFAULT_WIDTHS = (16, 32, 32, 8)
_FWD, _DX, _G = ProductKind.FORWARD, ProductKind.INPUT_GRAD, ProductKind.WEIGHT_GRAD


def _layer_dims(widths: Sequence[int]) -> Iterator[tuple[int, int, int]]:
    """``(ℓ, in, out)`` for ``ℓ = 1..L``."""
    for l in range(1, len(widths)):
        yield l, widths[l - 1], widths[l]


class MLP(nn.Module):
    """The ``tanh`` MLP; ``forward`` gives ``Y_L``. Building it draws nothing from the global
    random state (its initial weights are overwritten by the step's ``W_t``)."""

    def __init__(self, widths: Sequence[int]) -> None:
        super().__init__()
        with torch.random.fork_rng(devices=[]):
            self.layers = nn.ModuleList([nn.Linear(i, o, bias=False)
                                         for _, i, o in _layer_dims(widths)])
        self.act = nn.Tanh()
        self.loss_fn = nn.MSELoss(reduction="mean")

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        *hidden, last = self.layers
        for layer in hidden:
            x = self.act(layer(x))
        return last(x)


def make_record(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """The record of one example: ``x ‖ y`` as a new contiguous float32 vector."""
    if x.dim() != 1 or y.dim() != 1:
        raise ValueError("x and y must be 1-D")
    out = torch.empty(x.numel() + y.numel(), dtype=torch.float32)
    out[:x.numel()] = x
    out[x.numel():] = y
    return out


def split_record(record: torch.Tensor, d_in: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``(x, y)`` views of a record, or of records stacked along the first dimension."""
    return record.narrow(-1, 0, d_in), record.narrow(-1, d_in, record.shape[-1] - d_in)


def init_weights(widths: Sequence[int], seed: int,
                 device: torch.device | str = "cpu") -> dict[str, torch.Tensor]:
    """A seeded ``W_0``: layer ``ℓ``'s entries uniform on ``[−1/√i, 1/√i)``, the range
    ``nn.Linear`` draws from, layer after layer from one generator."""
    g = torch.Generator().manual_seed(seed)
    out = {}
    for l, i, o in _layer_dims(widths):
        bound = 1.0 / math.sqrt(i)
        w = torch.empty(o, i).uniform_(-bound, bound, generator=g)
        out[f"layers.{l - 1}.weight"] = w.to(device)
    return out


def synthetic_dataset(widths: Sequence[int], n_records: int, seed: int) -> list[torch.Tensor]:
    """``n_records`` host records: inputs ``N(0, 1)``, targets from a teacher MLP with its own
    seeded weights, so the task is learnable."""
    g = torch.Generator().manual_seed(seed)
    inputs = torch.randn(n_records, widths[0], generator=g)
    teacher = MLP(widths)
    load_weights(_Names(widths), teacher, init_weights(widths, seed + 1))
    with torch.no_grad():
        targets = teacher(inputs)
    return [make_record(x, y) for x, y in zip(inputs, targets)]


class _Names:
    """The weight names of an MLP of these widths, as ``load_weights`` reads them."""

    def __init__(self, widths: Sequence[int]) -> None:
        self.weight_names = tuple(f"layers.{l - 1}.weight" for l, _, _ in _layer_dims(widths))


class MLPComputation(DeclaredComputation):
    """``C`` for the MLP at ``widths``, ``n_s`` records a step, SGD step size ``eta``."""

    def __init__(self, widths: Sequence[int] = DEFAULT_WIDTHS, n_s: int = 4, *,
                 eta: float) -> None:
        widths = tuple(int(w) for w in widths)
        if len(widths) < 2:
            raise ValueError("need at least one layer")
        # q is a width (Y, dX) or n_s (G); a q = 1 product is glue, not a checked matmul
        if n_s < 2 or min(widths) < 2:
            raise ValueError(f"n_s={n_s} and widths={widths} must all be at least 2")
        if not (isinstance(eta, float) and 0 < eta < math.inf):
            raise ValueError(f"eta must be a positive finite float, got {eta!r}")
        self.widths, self.L, self._n_s, self._eta = widths, len(widths) - 1, int(n_s), eta
        self.validate()

    @property
    def n_s(self) -> int:
        return self._n_s

    @property
    def eta(self) -> float:
        return self._eta

    @property
    def d_in(self) -> int:
        return self.widths[0]

    @property
    def d_out(self) -> int:
        return self.widths[-1]

    @cached_property
    def weight_names(self) -> tuple[str, ...]:
        return _Names(self.widths).weight_names

    def weight(self, l: int) -> str:
        """The name of ``W_ℓ`` (``ℓ`` from 1)."""
        return self.weight_names[l - 1]

    @cached_property
    def weight_shapes(self) -> dict[str, tuple[int, int]]:
        return {self.weight(l): (o, i) for l, i, o in _layer_dims(self.widths)}

    @cached_property
    def products(self) -> tuple[ProductSpec, ...]:
        n = self.n_s
        dims = {l: (i, o) for l, i, o in _layer_dims(self.widths)}
        table = [("Y", _FWD, l) for l in dims]
        for l in reversed(dims):
            table += ([("dX", _DX, l)] if l > 1 else []) + [("G", _G, l)]
        shapes = {_FWD: lambda i, o: ((n, i), (i, o)), _DX: lambda i, o: ((n, o), (o, i)),
                  _G: lambda i, o: ((o, n), (n, i))}
        return tuple(ProductSpec(m, f"{role}_{l}", kind, *shapes[kind](*dims[l]),
                                 weight=self.weight(l), layer=l)
                     for m, (role, kind, l) in enumerate(table, start=1))

    @cached_property
    def _by_name(self) -> dict[str, ProductSpec]:
        return {spec.name: spec for spec in self.products}

    def m_of(self, name: str) -> int:
        return self._by_name[name].m

    @cached_property
    def linear_weights(self) -> dict[str, tuple[int, ...]]:
        return {self.weight(l): (self.m_of(f"G_{l}"),) for l in range(1, self.L + 1)}

    # ---- records ----------------------------------------------------------------------------

    def _check_record(self, record: Any) -> None:
        width = self.d_in + self.d_out
        ok = isinstance(record, torch.Tensor) and record.dtype == torch.float32 \
            and tuple(record.shape) == (width,)
        if not ok:
            got = (getattr(record, "dtype", type(record).__name__),
                   tuple(getattr(record, "shape", ())))
            raise ValueError(f"an MLP record is a float32 [{width}] tensor, got "
                             f"{got[0]} {got[1]}")

    def encode_record(self, record: torch.Tensor) -> bytes:
        self._check_record(record)
        return encode_tensor_leaf(TAG_MLP_RECORD, record)

    def record_leaf(self, record: torch.Tensor) -> tuple[int, torch.Tensor]:
        self._check_record(record)
        return TAG_MLP_RECORD, record

    def assemble(self, records: Sequence[torch.Tensor],
                 device: torch.device | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """The batch glue: records stacked in batch order, split into ``(X_1, targets)``."""
        if len(records) != self.n_s:
            raise ValueError(f"batch has {len(records)} records, the computation declares "
                             f"{self.n_s}")
        for record in records:
            self._check_record(record)
        batch = torch.stack(list(records))
        if device is not None:
            batch = batch.to(device)
        x, y = split_record(batch, self.d_in)
        return x.contiguous(), y.contiguous()

    def build_model(self) -> MLP:
        return MLP(self.widths)

    def replay(self, leaves: Any) -> MLPReplay:
        given = getattr(self, "_operands", None)
        return given if given is not None else MLPReplay(self, leaves)

    # ---- prover side ----------------------------------------------------------------------

    def loss(self, model: nn.Module, records: Sequence[torch.Tensor]) -> torch.Tensor:
        x, targets = self.assemble(records, next(model.parameters()).device)
        return model.loss_fn(model(x), targets)

    def label(self, capture: Any, model: nn.Module) -> list[torch.Tensor]:
        """The captured products in canonical order, each recognised by its operands
        (reference mlp.py:242-291): a forward product reads ``W_ℓᵀ``; an input gradient reads
        ``W_ℓ``; a weight gradient reads ``X_ℓ`` (the storage ``Y_ℓ`` read as its input) and
        writes the storage autograd then holds as ``W_ℓ.grad``."""
        if capture.glue_outer:
            raise LabelingError(f"unexpected q=1 products: {len(capture.glue_outer)}")
        weight_layer = {name: l for l, name in enumerate(self.weight_names, start=1)}
        input_layer: dict[int, int] = {}  # storage of X_ℓ -> ℓ, from the forward records
        found: dict[str, torch.Tensor] = {}

        def slot_of(rec: Any) -> str:
            if rec.batch is not None:
                raise LabelingError(f"record #{rec.index}: the MLP has no batched products")
            if rec.a is None:
                raise LabelingError("the capture's operands were released before labeling")
            by_weight = weight_layer.get(rec.b_info.param_name)
            if rec.phase == "forward":
                if by_weight is None:
                    raise LabelingError(f"forward record #{rec.index} has no weight operand")
                if input_layer.setdefault(rec.a_info.storage_ptr, by_weight) != by_weight:
                    raise LabelingError(f"forward record #{rec.index}: X_{by_weight} aliases "
                                        f"another input")
                return f"Y_{by_weight}"
            if by_weight is not None:
                return f"dX_{by_weight}"
            l = input_layer.get(rec.b_info.storage_ptr)
            if l is None:
                raise LabelingError(f"backward record #{rec.index} matches no declared slot")
            grad = model.get_parameter(self.weight(l)).grad
            if grad is None or not capture.is_output_of(grad, rec):
                raise LabelingError(f"G_{l} (record #{rec.index}) is not W_{l}.grad")
            return f"G_{l}"

        # forward records first: a weight gradient is recognised by a forward input
        ordered = sorted(capture.records, key=lambda r: r.phase != "forward")
        for rec in ordered:
            name = slot_of(rec)
            spec = self._by_name.get(name)
            if spec is None:
                raise LabelingError(f"record #{rec.index} names no declared slot ({name})")
            if name in found:
                raise LabelingError(f"slot {name} filled twice (record #{rec.index})")
            shapes = (tuple(rec.a.shape), tuple(rec.b.shape), tuple(rec.out.shape))
            if shapes != (spec.a_shape, spec.b_shape, spec.p_shape):
                raise LabelingError(f"{name}: shapes {shapes} != declared "
                                    f"{(spec.a_shape, spec.b_shape, spec.p_shape)}")
            found[name] = rec.out
        missing = [spec.name for spec in self.products if spec.name not in found]
        if missing:
            raise LabelingError(f"slots never filled: {missing}")
        return [found[spec.name] for spec in self.products]


class MLPReplay(Replay):
    """The verifier's glue for one MLP step, from the committed leaves, on the GPU.

    ``leaves`` is anything with ``leaf(index)`` (check 5 passes the leaves check 2 hashed) or
    a list. A model loaded from the committed ``W_t`` supplies ``act`` and ``loss_fn``. Each
    layer's ``X_ℓ`` and ``δY_ℓ`` is computed on first use and dropped after ``G_ℓ``, the last
    product in canonical order that reads them; asked again, it is recomputed from the leaves
    to the same values.
    """

    def __init__(self, computation: MLPComputation, leaves: Any,
                 device: torch.device | str | None = None) -> None:
        self.c, self.leaves = computation, leaves
        if device is None:
            device = torch.device("cuda", torch.cuda.current_device()) \
                if torch.cuda.is_available() else "cpu"
        self.device = torch.device(device)
        with self.device:
            self.model = computation.build_model()
        load_weights(computation, self.model,
                     {name: self.w_t(name) for name in computation.weight_names})
        n = computation.L + 2
        self._x: list[torch.Tensor | None] = [None] * n
        self._dy: list[torch.Tensor | None] = [None] * n
        self._batch: tuple[torch.Tensor, torch.Tensor] | None = None
        self._finished = False

    def _get(self, index: int) -> Any:
        reader = getattr(self.leaves, "leaf", None)
        obj = reader(index) if reader is not None else self.leaves[index]
        return obj.to(self.device) if isinstance(obj, torch.Tensor) else obj

    def w_t(self, name: str) -> torch.Tensor:
        return self._get(self.c.w_t_index(name))

    def product(self, name: str) -> torch.Tensor:
        return self._get(self.c.product_index(self.c.m_of(name)))

    def _records(self) -> tuple[torch.Tensor, torch.Tensor]:
        if self._batch is None:
            self._batch = self.c.assemble([self._get(i) for i in range(self.c.n_s)],
                                          self.device)
        return self._batch

    def x(self, l: int) -> torch.Tensor:
        """``X_ℓ``: the batch for ``ℓ = 1``, else ``tanh`` of the committed ``Y_{ℓ−1}``."""
        if self._x[l] is None:
            if l == 1:
                self._x[l] = self._records()[0]
            else:
                with torch.no_grad():
                    self._x[l] = self.model.act(self.product(f"Y_{l - 1}"))
        return self._x[l]

    def dy(self, l: int) -> torch.Tensor:
        """``δY_ℓ``, by autograd through ``loss_fn`` (the last layer) or ``act``."""
        if self._dy[l] is None:
            y = self.product(f"Y_{l}").detach().requires_grad_(True)
            with torch.enable_grad():
                if l == self.c.L:
                    out, seed = self.model.loss_fn(y, self._records()[1]), None
                else:
                    out, seed = self.model.act(y), self.product(f"dX_{l + 1}")
                self._dy[l] = torch.autograd.grad(out, y, grad_outputs=seed)[0].detach()
        return self._dy[l]

    def operands(self, m: int) -> tuple[torch.Tensor, torch.Tensor]:
        spec = self.c.product(m)
        l, w = spec.layer, self.w_t(spec.weight)
        if spec.kind is _FWD:
            pair = (self.x(l), w.t())
        elif spec.kind is _DX:
            pair = (self.dy(l), w)
        else:  # G_ℓ, the last reader of this layer's glue
            pair = (self.dy(l).t(), self.x(l))
            self._x[l] = self._dy[l] = None
        self._finished |= m == self.c.M
        return pair

    def glue_gradients(self) -> dict[str, torch.Tensor]:
        """None: every MLP weight is linear and checked by 6a. Valid after ``operands(M)``."""
        if not self._finished:
            raise RuntimeError("glue_gradients is valid only after operands(M)")
        return {}
