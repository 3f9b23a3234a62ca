"""The MLP instance of the declared computation (reference:
verification/computation/instances/mlp.py:1-365), with its replay on the GPU.

Model: ``Y_ℓ = X_ℓ·W_ℓᵀ`` for ``ℓ = 1..L`` (bias-free linears), ``X_{ℓ+1} = tanh(Y_ℓ)`` for
``ℓ < L``, and the mean-squared-error loss of ``Y_L`` against the targets; ``L = len(widths) −
1``. ``X_1`` is batch data, so there is no ``δX_1`` and ``M = 3L − 1``.

The reference's pins, kept:

- **Record.** One batch record is a float32 ``[d_in + d_out]`` tensor, the input row then the
  target row. Its leaf is the tensor leaf with tag ``0x04``.
- **Canonical order.** Forward ``Y_1 … Y_L``, then for ``ℓ = L … 1`` the input gradient
  ``dX_ℓ`` (for ``ℓ ≥ 2``) and the weight gradient ``G_ℓ``.
- **Weights** ``layers.{ℓ−1}.weight``, ``[o, i]``, ``ℓ = 1..L``. Every weight is linear: check
  6a covers all of them, through ``G_ℓ``.

| product | A | B | P |
|---|---|---|---|
| ``Y_ℓ`` | ``X_ℓ`` | ``W_ℓᵀ`` | ``n_s × o`` |
| ``dX_ℓ`` | ``δY_ℓ`` | ``W_ℓ`` | ``n_s × i`` |
| ``G_ℓ`` | ``δY_ℓᵀ`` | ``X_ℓ`` | ``o × i`` |

with ``δY_L = ∂loss/∂Y_L`` and ``δY_ℓ = dX_{ℓ+1} ⊙ tanh′(Y_ℓ)``.

:class:`MLPReplay` rebuilds every operand from the committed leaves on the GPU: ``X_1`` and the
targets from the records, ``X_{ℓ+1} = tanh(Y_ℓ)`` from the committed ``Y_ℓ``, ``δY_ℓ`` by
autograd through the model's own ``loss_fn`` and ``act`` from the committed ``Y_ℓ`` and
``dX_{ℓ+1}``, the weights from ``W_t``. The glue is PyTorch; the operands go to the Freivalds
kernels as they are (``W_ℓᵀ`` and ``δY_ℓᵀ`` are transposed views).
"""

from __future__ import annotations

import math
from collections.abc import Sequence
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


class MLP(nn.Module):
    """``tanh`` MLP of bias-free linears; ``forward`` returns ``Y_L``. Construction leaves the
    global random state alone; load weights before use."""

    def __init__(self, widths: Sequence[int]) -> None:
        super().__init__()
        with torch.random.fork_rng(devices=[]):
            self.layers = nn.ModuleList(nn.Linear(i, o, bias=False)
                                        for i, o in zip(widths[:-1], widths[1:]))
        self.act = nn.Tanh()
        self.loss_fn = nn.MSELoss(reduction="mean")

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        last = len(self.layers) - 1
        for l, layer in enumerate(self.layers):
            x = layer(x)
            if l < last:
                x = self.act(x)
        return x


def make_record(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """One record ``x ‖ y``, a contiguous float32 vector."""
    if x.dim() != 1 or y.dim() != 1:
        raise ValueError("x and y must be 1-D")
    return torch.cat([x, y]).to(torch.float32).contiguous()


def split_record(record: torch.Tensor, d_in: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``(x, y)`` of one record or of a stacked batch."""
    return record[..., :d_in], record[..., d_in:]


def init_weights(widths: Sequence[int], seed: int,
                 device: torch.device | str = "cpu") -> dict[str, torch.Tensor]:
    """Seeded ``W_0``, entries uniform in ``(−1/√i, 1/√i)`` as ``nn.Linear`` draws them."""
    g = torch.Generator().manual_seed(seed)
    out = {}
    for l, (i, o) in enumerate(zip(widths[:-1], widths[1:])):
        bound = 1.0 / math.sqrt(i)
        out[f"layers.{l}.weight"] = ((torch.rand(o, i, generator=g) * 2 - 1) * bound).to(device)
    return out


def synthetic_dataset(widths: Sequence[int], n_records: int, seed: int) -> list[torch.Tensor]:
    """Records with ``x ~ N(0, 1)`` and ``y`` from a seeded teacher MLP (host tensors)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n_records, widths[0], generator=g)
    teacher = MLP(widths)
    with torch.no_grad():
        for name, w in init_weights(widths, seed + 1).items():
            teacher.get_parameter(name).copy_(w)
        y = teacher(x)
    return [make_record(x[i], y[i]) for i in range(n_records)]


class MLPComputation(DeclaredComputation):
    """The computation of :class:`MLP` at ``widths``, ``n_s`` records a step, step size
    ``eta``."""

    def __init__(self, widths: Sequence[int] = DEFAULT_WIDTHS, n_s: int = 4, *,
                 eta: float) -> None:
        widths = tuple(int(w) for w in widths)
        if len(widths) < 2:
            raise ValueError("need at least one layer")
        if n_s < 2 or min(widths) < 2:  # a q = 1 product would be glue, not a checked matmul
            raise ValueError(f"n_s={n_s} and widths={widths} must all be at least 2")
        if not (isinstance(eta, float) and 0 < eta < math.inf):
            raise ValueError(f"eta must be a positive finite float, got {eta!r}")
        self.widths = widths
        self.L = len(widths) - 1
        self._n_s = int(n_s)
        self._eta = eta
        self._names = tuple(f"layers.{l}.weight" for l in range(self.L))
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

    @property
    def weight_names(self) -> tuple[str, ...]:
        return self._names

    def weight(self, l: int) -> str:
        """``W_ℓ``'s name, ``ℓ`` 1-based."""
        return self._names[l - 1]

    @cached_property
    def weight_shapes(self) -> dict[str, tuple[int, int]]:
        return {self.weight(l): (self.widths[l], self.widths[l - 1])
                for l in range(1, self.L + 1)}

    @cached_property
    def products(self) -> tuple[ProductSpec, ...]:
        n, w = self.n_s, self.widths
        rows: list[tuple[str, ProductKind, tuple[int, int], tuple[int, int], int]] = []
        for l in range(1, self.L + 1):
            rows.append((f"Y_{l}", ProductKind.FORWARD, (n, w[l - 1]), (w[l - 1], w[l]), l))
        for l in range(self.L, 0, -1):
            i, o = w[l - 1], w[l]
            if l >= 2:
                rows.append((f"dX_{l}", ProductKind.INPUT_GRAD, (n, o), (o, i), l))
            rows.append((f"G_{l}", ProductKind.WEIGHT_GRAD, (o, n), (n, i), l))
        return tuple(ProductSpec(m, name, kind, a, b, weight=self.weight(l), layer=l)
                     for m, (name, kind, a, b, l) in enumerate(rows, start=1))

    @cached_property
    def _m_by_name(self) -> dict[str, int]:
        return {p.name: p.m for p in self.products}

    def m_of(self, name: str) -> int:
        return self._m_by_name[name]

    @cached_property
    def linear_weights(self) -> dict[str, tuple[int, ...]]:
        return {self.weight(l): (self.m_of(f"G_{l}"),) for l in range(1, self.L + 1)}

    def encode_record(self, record: torch.Tensor) -> bytes:
        self._check_record(record)
        return encode_tensor_leaf(TAG_MLP_RECORD, record)

    def record_leaf(self, record: torch.Tensor) -> tuple[int, torch.Tensor]:
        self._check_record(record)
        return TAG_MLP_RECORD, record

    def _check_record(self, record: Any) -> None:
        if (not isinstance(record, torch.Tensor) or record.dtype != torch.float32
                or tuple(record.shape) != (self.d_in + self.d_out,)):
            raise ValueError(
                f"an MLP record is a float32 [{self.d_in + self.d_out}] tensor, got "
                f"{getattr(record, 'dtype', type(record))} "
                f"{tuple(getattr(record, 'shape', ()))}")

    def assemble(self, records: Sequence[torch.Tensor],
                 device: torch.device | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """Glue: the records stacked in batch order and split into ``(X_1, targets)``."""
        if len(records) != self.n_s:
            raise ValueError(f"batch has {len(records)} records, the computation declares "
                             f"{self.n_s}")
        for r in records:
            self._check_record(r)
        batch = torch.stack([r if device is None else r.to(device) for r in records])
        x, y = split_record(batch, self.d_in)
        return x.contiguous(), y.contiguous()

    def build_model(self) -> MLP:
        return MLP(self.widths)

    # ---- verifier side --------------------------------------------------------------------

    def replay(self, leaves: Any) -> MLPReplay:
        if getattr(self, "_operands", None) is not None:
            return self._operands
        return MLPReplay(self, leaves)

    # ---- prover side ----------------------------------------------------------------------

    def loss(self, model: nn.Module, records: Sequence[torch.Tensor]) -> torch.Tensor:
        dev = next(model.parameters()).device
        x, targets = self.assemble(records, dev)
        return model.loss_fn(model(x), targets)

    def label(self, capture: Any, model: nn.Module) -> list[torch.Tensor]:
        """Map the captured records to slots by operand identity (reference mlp.py:242-291):
        a forward product's ``B`` views ``W_ℓ``; an input gradient's ``B`` is ``W_ℓ``; a weight
        gradient's ``B`` is ``X_ℓ``, the storage of ``Y_ℓ``'s ``A``, and its output is the
        storage AccumulateGrad adopted as ``W_ℓ.grad``."""
        if capture.glue_outer:
            raise LabelingError(f"unexpected q=1 products: {len(capture.glue_outer)}")
        layer = {n: l for l, n in enumerate(self.weight_names, start=1)}
        slots: dict[str, torch.Tensor] = {}
        x_of: dict[int, int] = {}  # storage of X_ℓ (a forward A) -> ℓ

        def fill(name: str, rec) -> None:
            if name in slots:
                raise LabelingError(f"slot {name} filled twice (record #{rec.index})")
            spec = self.product(self.m_of(name))
            got = (tuple(rec.a.shape), tuple(rec.b.shape), tuple(rec.out.shape))
            want = (spec.a_shape, spec.b_shape, spec.p_shape)
            if got != want:
                raise LabelingError(f"{name}: shapes {got} != declared {want}")
            slots[name] = rec.out

        for rec in capture.records:
            if rec.batch is not None:
                raise LabelingError(f"record #{rec.index}: the MLP has no batched products")
            if rec.a is None:
                raise LabelingError("the capture's operands were released before labeling")
        for rec in (r for r in capture.records if r.phase == "forward"):
            l = layer.get(rec.b_info.param_name)
            if l is None:
                raise LabelingError(f"forward record #{rec.index} has no weight operand")
            if rec.a_info.storage_ptr in x_of:
                raise LabelingError(f"forward record #{rec.index}: X_{l} aliases another input")
            x_of[rec.a_info.storage_ptr] = l
            fill(f"Y_{l}", rec)
        for rec in (r for r in capture.records if r.phase == "backward"):
            if rec.b_info.param_name in layer:
                fill(f"dX_{layer[rec.b_info.param_name]}", rec)
            elif rec.b_info.storage_ptr in x_of:
                l = x_of[rec.b_info.storage_ptr]
                grad = model.get_parameter(self.weight(l)).grad
                if grad is None or not capture.is_output_of(grad, rec):
                    raise LabelingError(f"G_{l} (record #{rec.index}) is not W_{l}.grad")
                fill(f"G_{l}", rec)
            else:
                raise LabelingError(f"backward record #{rec.index} matches no declared slot")
        missing = [p.name for p in self.products if p.name not in slots]
        if missing:
            raise LabelingError(f"slots never filled: {missing}")
        return [slots[p.name] for p in self.products]


class MLPReplay(Replay):
    """The glue replay of one MLP step from its committed leaves, on the GPU.

    ``leaves`` is anything with ``leaf(index)`` (check 5 passes the leaves check 2 hashed; a
    list works too). The replay owns an :class:`MLP` loaded from the committed ``W_t``, whose
    ``act`` and ``loss_fn`` run the glue. ``X_ℓ`` and ``δY_ℓ`` are kept from their first use to
    ``G_ℓ``, their last consumer in canonical order; any other order recomputes them from the
    leaves and gives the same operands.
    """

    def __init__(self, computation: MLPComputation, leaves: Any,
                 device: torch.device | str | None = None) -> None:
        self.c = computation
        self.leaves = leaves
        if device is None:
            device = torch.device("cuda", torch.cuda.current_device()) \
                if torch.cuda.is_available() else torch.device("cpu")
        self.device = torch.device(device)
        with self.device:  # the parameters are created (and initialised) on the device
            self.model = computation.build_model()
        load_weights(computation, self.model,
                     {n: self.w_t(n) for n in computation.weight_names})
        self._x: dict[int, torch.Tensor] = {}
        self._dy: dict[int, torch.Tensor] = {}
        self._targets: torch.Tensor | None = None
        self._done = False

    def _leaf(self, index: int) -> Any:
        get = getattr(self.leaves, "leaf", None)
        obj = get(index) if get is not None else self.leaves[index]
        return obj.to(self.device) if isinstance(obj, torch.Tensor) else obj

    def w_t(self, name: str) -> torch.Tensor:
        return self._leaf(self.c.w_t_index(name))

    def product(self, name: str) -> torch.Tensor:
        return self._leaf(self.c.product_index(self.c.m_of(name)))

    def _batch(self) -> tuple[torch.Tensor, torch.Tensor]:
        records = [self._leaf(i) for i in range(self.c.n_s)]
        x1, targets = self.c.assemble(records, self.device)
        self._targets = targets
        return x1, targets

    def x(self, l: int) -> torch.Tensor:
        """``X_ℓ``: the batch for ``ℓ = 1``, else ``tanh`` of the committed ``Y_{ℓ−1}``."""
        if l not in self._x:
            if l == 1:
                self._x[l] = self._batch()[0]
            else:
                with torch.no_grad():
                    self._x[l] = self.model.act(self.product(f"Y_{l - 1}"))
        return self._x[l]

    def dy(self, l: int) -> torch.Tensor:
        """``δY_ℓ`` by autograd through the model's ``loss_fn`` (``ℓ = L``) or ``act``."""
        if l not in self._dy:
            y = self.product(f"Y_{l}").detach().requires_grad_(True)
            with torch.enable_grad():
                if l == self.c.L:
                    targets = self._targets if self._targets is not None else self._batch()[1]
                    (g,) = torch.autograd.grad(self.model.loss_fn(y, targets), y)
                else:
                    upstream = self.product(f"dX_{l + 1}")
                    (g,) = torch.autograd.grad(self.model.act(y), y, grad_outputs=upstream)
            self._dy[l] = g.detach()
        return self._dy[l]

    def operands(self, m: int) -> tuple[torch.Tensor, torch.Tensor]:
        spec = self.c.product(m)
        l = spec.layer
        w = self.w_t(spec.weight)
        if spec.kind is ProductKind.FORWARD:
            out = self.x(l), w.t()
        elif spec.kind is ProductKind.INPUT_GRAD:
            out = self.dy(l), w
        else:
            out = self.dy(l).t(), self.x(l)
            self._x.pop(l, None)
            self._dy.pop(l, None)
        if m == self.c.M:
            self._done = True
        return out

    def glue_gradients(self) -> dict[str, torch.Tensor]:
        """Every MLP weight is linear (check 6a), so there are no glue gradients."""
        if not self._done:
            raise RuntimeError("glue_gradients is valid only after operands(M)")
        return {}
