"""A synthetic training-step transcript, resident in HBM, for benchmarks and tests.

Reference: the transcript the prover commits (verification/prover/step.py:171-269) holds the
batch records, ``W_t``, every matmul output ``P_m`` and ``W_{t+1}`` in the layout of the
declared computation. This module builds one with the declared shapes and dtypes without
running the model: each product's operands ``A_m, B_m`` are drawn i.i.d. normal (``B`` scaled
by ``1/√q`` so ``P`` stays O(1)), in the compute dtype, and ``P_m = A_m·B_m (+ 1·bᵀ)`` is
computed by torch on the GPU with fp32 accumulation and rounded to the compute dtype, as a
bf16-autocast step stores it. The members of one batched attention product (one layer and
role, ``c.operand_groups``) are generated and multiplied as one stack, as a step holds them,
and the replay serves each such group as that stack (``operand_group``). A linear weight's
``W_{t+1}`` is ``W_t − η·G`` with ``G`` the chain of its committed weight-gradient products
(so check 6a holds), a glue weight's moves by a random step. Where the computation names operand twins (``operand_twins``: products
whose A is, in a real step, the transpose of an earlier product's A), the later product's A
is that tensor transposed, and its P is the fp32 sum rounded to the compute dtype.

The verifier's work per product (hash the leaf, measure ``A(B·r) − P·r``) depends only on
shapes and dtypes, so the timings equal a real step's; the values are not a trained model's.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from setup.records import Record
from verification.computation.interface import DeclaredComputation, Replay, chain_gradient


@dataclass
class SyntheticStep:
    c: DeclaredComputation
    leaves: list
    operands: dict[int, tuple[torch.Tensor, torch.Tensor]] = field(default_factory=dict)
    # the stacked operands of each group of batched members: {ms: (A [g, n, q], B [g, q, w])}
    groups: dict[tuple[int, ...], tuple[torch.Tensor, torch.Tensor]] = \
        field(default_factory=dict)

    def product(self, m: int) -> torch.Tensor:
        return self.leaves[self.c.product_index(m)]

    def w_t(self, name: str) -> torch.Tensor:
        return self.leaves[self.c.w_t_index(name)]

    def replay(self) -> CapturedReplay:
        """The captured operands as check 5's operand source."""
        return CapturedReplay(self.operands, self.groups)


class CapturedReplay(Replay):
    """Check 5's operands as the prover used them: ``operands[m] = (A_m, B_m)``. They come
    from the prover, not from the committed leaves, so a verifier takes them only when told
    to trust them (``prover_supplied``). ``groups`` holds the whole operands of batched
    products (``{ms: (A, B)}`` with ``A[i], B[i]`` product ``ms[i]``'s), which
    :meth:`operand_group` serves as they lie."""

    prover_supplied = True

    def __init__(self, operands: dict[int, tuple[torch.Tensor, torch.Tensor]],
                 groups: dict[tuple[int, ...], tuple[torch.Tensor, torch.Tensor]]
                 | None = None) -> None:
        self._ops = operands
        self._groups = groups or {}

    def operands(self, m: int) -> tuple[torch.Tensor, torch.Tensor]:
        try:
            return self._ops[m]
        except KeyError:
            raise IndexError(f"no captured operands for product m={m}") from None

    def operand_group(self, ms, dtype=None):
        got = self._groups.get(tuple(ms))
        if got is None or dtype is not None:
            return super().operand_group(ms, dtype)
        for m in ms:  # the same first error as serving member by member
            self.operands(m)
        return got


def _stack_of(parts: list[tuple[torch.Tensor, int]]) -> tuple[torch.Tensor, int] | None:
    """``(stack, first index)`` when ``parts`` are consecutive members of one stack."""
    stack, i0 = parts[0]
    if all(s is stack and i == i0 + j for j, (s, i) in enumerate(parts)):
        return stack, i0
    return None


@torch.no_grad()
def synthetic_step(c: DeclaredComputation, *, seed: int = 0, device: str = "cuda",
                   operands: bool = True, eta: float = 1e-4) -> SyntheticStep:
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    cg = torch.Generator().manual_seed(seed)
    dt = c.product_dtype
    leaves: list = []
    n_tok = getattr(c, "n", 16)
    n_v = getattr(c, "n_v", 1000)
    for _ in range(c.n_s):
        ids = torch.randint(0, n_v, (n_tok,), generator=cg, dtype=torch.int32)
        leaves.append(Record(ids, torch.roll(ids, -1), torch.ones(n_tok, dtype=torch.int32)))
    w_t = {}
    for name in c.weight_names:
        shape = c.weight_shapes[name]
        w = torch.randn(shape, generator=g, device=dev, dtype=torch.float32)
        w.mul_(0.02 if len(shape) == 2 else 1.0)
        w_t[name] = w
        leaves.append(w)
    ops: dict[int, tuple[torch.Tensor, torch.Tensor]] = {}
    groups: dict[tuple[int, ...], tuple[torch.Tensor, torch.Tensor]] = {}
    # A product whose A is, in a real step, the transpose of an earlier product's A (dV of O's
    # attention probabilities, dK of dQ's δS, G of dX's output gradient) gets that very tensor,
    # transposed, as its A: the verifier's reads depend on which operands alias.
    twins = getattr(c, "operand_twins", None) or {}
    need = set(twins.values())
    firsts: dict[int, tuple[torch.Tensor, int]] = {}  # m → (its A's stack, its index)
    p_leaves: list[torch.Tensor | None] = [None] * c.M
    # The members of one batched product are generated as one stack, as a step holds them.
    for grp in c.operand_groups:
        specs = [c.products[i] for i in grp]
        s0 = specs[0]
        (n, q), (_, w) = s0.a_shape, s0.b_shape
        k = len(specs)
        ms = tuple(s.m for s in specs)
        if s0.m in twins:
            b = torch.randn(k, q, w, generator=g, device=dev, dtype=torch.float32)
            b = b.mul_(q ** -0.5).to(dt)
            at = _stack_of([firsts.pop(twins[m]) for m in ms])
            if at is None:
                raise RuntimeError(f"{s0.name}: the twins' mates are not one stack")
            stack, i0 = at
            a = stack[i0:i0 + k].transpose(1, 2)
            # fp32 sums rounded to the compute dtype, as the bf16 products are
            ps = [torch.matmul(a[i].float(), b[i].float()).to(dt) for i in range(k)]
        else:
            a = torch.randn(k, n, q, generator=g, device=dev, dtype=torch.float32).to(dt)
            b = torch.randn(k, q, w, generator=g, device=dev, dtype=torch.float32)
            b = b.mul_(q ** -0.5).to(dt)
            for i, m in enumerate(ms):
                if m in need:
                    firsts[m] = (a, i)
            if k == 1:
                acc = torch.matmul(a[0].float(), b[0].float()) if dt == torch.float32 else \
                    torch.matmul(a[0], b[0]).float()
                if s0.bias is not None:
                    acc += w_t[s0.bias].to(dt).float()
                ps = [acc.to(dt)]
            else:
                ps = list(torch.bmm(a, b).unbind(0))
        for i, idx in enumerate(grp):
            p_leaves[idx] = ps[i].contiguous()
        if operands:
            for i, m in enumerate(ms):
                ops[m] = (a[i], b[i])
            if k > 1:
                groups[ms] = (a, b)
        del a, b, ps
    leaves.extend(p_leaves)
    # W_{t+1}: a linear weight takes the SGD step from its committed gradient products, as
    # the optimizer writes it (``W_t.add(G, alpha=-η)``, check 6a's honest case); the other
    # (glue) weights move by a random step of the same size.
    try:
        eta = c.eta
    except NotImplementedError:
        pass
    linear = c.linear_weights
    for name in c.weight_names:
        w = w_t[name]
        if name in linear:
            grad = chain_gradient((leaves[c.product_index(m)] for m in linear[name]),
                                  torch.float32)
            leaves.append(torch.add(w, grad, alpha=-eta))
        else:
            leaves.append(w - eta * torch.randn(w.shape, generator=g, device=dev))
    return SyntheticStep(c, leaves, ops, groups)


@torch.no_grad()
def perturb_products(step: SyntheticStep, fraction: float = 0.01, *, seed: int = 0,
                     lo: float = 1e-6, hi: float = 1.0) -> list[tuple[int, int, float]]:
    """Adversarial products: a seeded ``fraction`` of the product leaves each get one seeded
    entry multiplied by ``1 ± x``, with ``x`` log-uniform in ``[lo, hi]`` (in place, in the
    leaf's own dtype). Returns ``(m, flat index, factor)`` per perturbed product, in canonical
    order. The transcript's root changes with it, as a prover committing the forged leaves
    would re-root."""
    import math
    c = step.c
    g = torch.Generator().manual_seed(seed)
    n = max(1, round(fraction * c.M))
    ms = sorted(int(x) + 1 for x in torch.randperm(c.M, generator=g)[:n])
    out = []
    for m in ms:
        p = step.product(m)
        idx = int(torch.randint(0, p.numel(), (1,), generator=g))
        u = float(torch.rand(1, generator=g))
        x = math.exp(math.log(lo) + u * (math.log(hi) - math.log(lo)))
        sign = 1.0 if float(torch.rand(1, generator=g)) < 0.5 else -1.0
        factor = 1.0 + sign * x
        flat = p.view(-1)
        flat[idx] = (flat[idx].float() * factor).to(p.dtype)
        out.append((m, idx, factor))
    return out
