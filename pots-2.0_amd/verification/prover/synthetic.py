"""A synthetic training-step transcript, resident in HBM, for benchmarks and tests.

Reference: the transcript the prover commits (verification/prover/step.py:171-269) holds the
batch records, ``W_t``, every matmul output ``P_m`` and ``W_{t+1}`` in the layout of the
declared computation. This module builds one with the declared shapes and dtypes without
running the model: each product's operands ``A_m, B_m`` are drawn i.i.d. normal (``B`` scaled
by ``1/√q`` so ``P`` stays O(1)), in the compute dtype, and ``P_m = A_m·B_m (+ 1·bᵀ)`` is
computed by torch on the GPU with fp32 accumulation and rounded to the compute dtype, as a
bf16-autocast step stores it. Attention members of one layer and role are generated and
multiplied as one stacked batch. A linear weight's ``W_{t+1}`` is ``W_t − η·G`` with ``G`` the
chain of its committed weight-gradient products (so check 6a holds), a glue weight's moves
by a random step. Where the computation names operand twins (``operand_twins``: products
whose A is, in a real step, the transpose of an earlier product's A), the later product's A
is that tensor transposed, and its P is the fp32 sum rounded to the compute dtype.

The verifier's work per product (hash the leaf, measure ``A(B·r) − P·r``) depends only on
shapes and dtypes, so the timings equal a real step's; the values are not a trained model's.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from setup.records import Record
from verification.computation.interface import (DeclaredComputation, ProductSpec, Replay,
                                               chain_gradient)


@dataclass
class SyntheticStep:
    c: DeclaredComputation
    leaves: list
    operands: dict[int, tuple[torch.Tensor, torch.Tensor]] = field(default_factory=dict)

    def product(self, m: int) -> torch.Tensor:
        return self.leaves[self.c.product_index(m)]

    def w_t(self, name: str) -> torch.Tensor:
        return self.leaves[self.c.w_t_index(name)]

    def replay(self) -> CapturedReplay:
        """The captured operands as check 5's operand source."""
        return CapturedReplay(self.operands)


class CapturedReplay(Replay):
    """Check 5's operands as the prover used them: ``operands[m] = (A_m, B_m)``. They come
    from the prover, not from the committed leaves, so a verifier takes them only when told
    to trust them (``prover_supplied``)."""

    prover_supplied = True

    def __init__(self, operands: dict[int, tuple[torch.Tensor, torch.Tensor]]) -> None:
        self._ops = operands

    def operands(self, m: int) -> tuple[torch.Tensor, torch.Tensor]:
        try:
            return self._ops[m]
        except KeyError:
            raise IndexError(f"no captured operands for product m={m}") from None


def _runs(c: DeclaredComputation) -> list[list[ProductSpec]]:
    """Consecutive products of one layer, member flag and shape pair, generated together."""
    out: list[list[ProductSpec]] = []
    for s in c.products:
        if out and s.member is not None and out[-1][0].member is not None \
                and out[-1][0].layer == s.layer and out[-1][0].a_shape == s.a_shape \
                and out[-1][0].b_shape == s.b_shape and out[-1][0].name.split("[")[0] \
                == s.name.split("[")[0]:
            out[-1].append(s)
        else:
            out.append([s])
    return out


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
    # A product whose A is, in a real step, the transpose of an earlier product's A (dV of O's
    # attention probabilities, dK of dQ's δS, G of dX's output gradient) gets that very tensor,
    # transposed, as its A: the verifier's reads depend on which operands alias.
    twins = getattr(c, "operand_twins", None) or {}
    firsts: dict[int, torch.Tensor] = {}
    need = set(twins.values())
    for run in _runs(c):
        s0 = run[0]
        (n, q), (_, w) = s0.a_shape, s0.b_shape
        k = len(run)
        if s0.m in twins:
            b = torch.randn(k, q, w, generator=g, device=dev, dtype=torch.float32)
            b = b.mul_(q ** -0.5).to(dt)
            for i, spec in enumerate(run):
                a = firsts.pop(twins[spec.m]).t()
                # fp32 sums rounded to the compute dtype, as the bf16 products are
                p = torch.matmul(a.float(), b[i].float())
                leaves.append(p.to(dt).contiguous())
                if operands:
                    ops[spec.m] = (a, b[i])
            del b
            continue
        a = torch.randn(k, n, q, generator=g, device=dev, dtype=torch.float32).to(dt)
        b = torch.randn(k, q, w, generator=g, device=dev, dtype=torch.float32)
        b = b.mul_(q ** -0.5).to(dt)
        for i, spec in enumerate(run):
            if spec.m in need:
                firsts[spec.m] = a[i]
        if k == 1:
            acc = torch.matmul(a[0].float(), b[0].float()) if dt == torch.float32 else \
                torch.matmul(a[0], b[0]).float()
            if s0.bias is not None:
                acc += w_t[s0.bias].to(dt).float()
            ps = [acc.to(dt)]
        else:
            ps = list(torch.bmm(a.contiguous(), b.contiguous()).unbind(0))
        for i, spec in enumerate(run):
            leaves.append(ps[i].contiguous())
            if operands:
                ops[spec.m] = (a[i], b[i])
        del a, b
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
    return SyntheticStep(c, leaves, ops)


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
