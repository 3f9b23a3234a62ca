"""Check 5's two tests on products ``P = A·B``, as numbers (reference:
verification/verifier/matmul_check/freivalds.py).

For one product, test 1 (the cancellation guard) compares ``ν = ‖|A|·(|B|·1)‖`` with
``‖|P|·1‖``; test 2 measures ``‖A(B·r_j) − P·r_j‖`` for ``k`` challenge vectors keyed on the
claimed root, against the band unit ``σ_r·e_m·‖P‖_F`` with ``e_m`` from the term scale
``U = sqrt(Σ_i (A²·(B²·1))_i)``. A bias ``P = A·B + 1·bᵀ`` is checked as ``[A | 1]·[B ; bᵀ]``.

Every number is computed on the GPU by ``libpots_mi355x`` (``native.FvPlan``): three streaming
passes read ``B``, ``A`` and ``P`` once each (matrix cores for the ``·R`` products, fp32
accumulation), and the norms are summed in fp64, which gives ``_safe_norm``'s semantics (a
finite norm when fp32 squares would overflow, 0 for a zero vector, a non-finite norm for a
non-finite input) without its power-of-two scaling. The rows are the reference's
:data:`ROW`, fp64 on the operands' device; :func:`finish_row` turns one row into a
:class:`ProductMeasure` on the host, with the reference's arithmetic.

Operands may be fp32 or bf16 (bf16 values are widened exactly, as the reference's
``.to(float32)``), on the GPU or the CPU (copied to the GPU). A product whose rows are not
unit-stride is made contiguous first.
"""

from __future__ import annotations

import math
from collections.abc import Sequence
from dataclasses import dataclass, replace

import numpy as np
import torch

from verification.commitment import native
from verification.verifier.matmul_check.challenges import SIGMA_R
from verification.verifier.matmul_check.sizing import product_e_m

__all__ = ["ROW", "MeasureScratch", "ProductMeasure", "RowArrays", "band_unit", "finish_row",
           "finish_rows", "finish_row_arrays",
           "measure_product", "measure_product_row", "measure_products",
           "measure_products_rows", "row_width", "term_scale", "term_scales",
           "measure_batch_rows"]


@dataclass(frozen=True)
class ProductMeasure:
    """Check 5's numbers for one product. Any of them may be non-finite; the caller judges."""

    nu: float
    p_abs1: float
    kappa: float
    residuals: tuple[float, ...]
    p_norm: float
    unit: float
    normalized: tuple[float, ...]
    u: float = math.nan


ROW = ("nu", "p_abs1", "p_norm", "u2_terms", "bias_sq", "residuals")
"""The columns of a product's fp64 row: ``ν``, ``‖|P|·1‖``, ``‖P‖_F``, ``Σ_i (A²·(B²·1))_i``,
``‖b‖²`` (0 without a bias), then the ``k`` residuals. ``ν`` and ``‖|P|·1‖`` are NaN when
test 1 is skipped."""


def row_width(k: int) -> int:
    return len(ROW) - 1 + k


class MeasureScratch:
    """Kept for the reference's signatures. The GPU plan owns its workspace, so this object
    holds nothing; passing one changes no number."""

    def __init__(self) -> None:
        pass


def _gpu(x: torch.Tensor) -> torch.Tensor:
    x = x.detach()
    if not x.is_cuda:
        x = x.to("cuda")
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.to(torch.float32)
    if x.dim() == 2 and x.stride(1) != 1:
        x = x.contiguous()
    return x


def measure_batch_rows(products: Sequence[tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                                torch.Tensor | None, int]],
                       *, h: bytes | torch.Tensor, k: int, guard: bool = True) -> torch.Tensor:
    """Rows of many products at once: ``(a, b, p, bias, m)`` each, one GPU plan, one pass per
    operand kind. Returns fp64 ``[len(products), 5 + k]`` on the GPU."""
    prods = [native.FvProduct(_gpu(a), _gpu(b), _gpu(p), m,
                              None if bias is None else _gpu(bias).float())
             for a, b, p, bias, m in products]
    plan = native.get().fv_plan(prods, k, guard)
    rows = plan.rows(h)
    torch.cuda.current_stream().synchronize()
    plan.close()
    return rows


def measure_product_row(a: torch.Tensor, b: torch.Tensor, p: torch.Tensor, *, h: bytes, m: int,
                        k: int, scratch: MeasureScratch | None = None, guard: bool = True,
                        bias: torch.Tensor | None = None) -> torch.Tensor:
    """:func:`measure_product`'s numbers as a fp64 row (:data:`ROW`) on the operands' device."""
    rows = measure_batch_rows([(a, b, p, bias, m)], h=h, k=k, guard=guard)
    return rows[0].to(a.device)


def measure_product(a: torch.Tensor, b: torch.Tensor, p: torch.Tensor, *, h: bytes, m: int,
                    k: int, eps_in: float, eps_acc: float,
                    scratch: MeasureScratch | None = None, guard: bool = True,
                    bias: torch.Tensor | None = None) -> ProductMeasure:
    """Both tests' numbers for product ``m``, challenges keyed on root ``h``."""
    row = measure_product_row(a, b, p, h=h, m=m, k=k, scratch=scratch, guard=guard, bias=bias)
    return finish_row(row.tolist(), q=a.shape[1] + (bias is not None), n=a.shape[0],
                      eps_in=eps_in, eps_acc=eps_acc, guard=guard, biased=bias is not None)


def measure_products_rows(a: torch.Tensor, b: torch.Tensor, p: torch.Tensor, *, h: bytes,
                          ms: Sequence[int], k: int, scratch: MeasureScratch | None = None,
                          guard: bool = True) -> torch.Tensor:
    """Rows ``[B, 5 + k]`` of a stacked batch ``p[i] = a[i]·b[i]`` (``[B, n, q]``,
    ``[B, q, w]``, ``[B, n, w]``), each member with its own challenges ``r(ms[i], j)``."""
    n_b = a.shape[0]
    if len(ms) != n_b or b.shape[0] != n_b or p.shape[0] != n_b:
        raise ValueError(f"batch of {len(ms)} labels for operands {tuple(a.shape)}, "
                         f"{tuple(b.shape)}, {tuple(p.shape)}")
    if n_b == 0:
        return torch.empty(0, 5 + k, dtype=torch.float64, device=a.device)
    rows = measure_batch_rows([(a[i], b[i], p[i], None, ms[i]) for i in range(n_b)], h=h, k=k,
                              guard=guard)
    return rows.to(a.device)


def measure_products(a: torch.Tensor, b: torch.Tensor, p: torch.Tensor, *, h: bytes,
                     ms: Sequence[int], k: int, eps_in: float, eps_acc: float,
                     scratch: MeasureScratch | None = None,
                     guard: bool = True) -> list[ProductMeasure]:
    """:func:`measure_product` for each member of a stacked batch."""
    rows = measure_products_rows(a, b, p, h=h, ms=ms, k=k, scratch=scratch, guard=guard)
    q, n = a.shape[2], a.shape[1]
    return [finish_row(row, q=q, n=n, eps_in=eps_in, eps_acc=eps_acc, guard=guard)
            for row in rows.tolist()]


def term_scale(a: torch.Tensor, b: torch.Tensor, bias: torch.Tensor | None = None) -> float:
    """``U`` of ``A·B`` (``[A | 1]·[B ; biasᵀ]`` given ``bias``)."""
    p = torch.zeros(a.shape[0], b.shape[1], dtype=torch.float32, device="cuda")
    row = measure_batch_rows([(a, b, p, bias, 1)], h=bytes(32), k=1)[0].tolist()
    u2 = row[3] + (a.shape[0] * row[4] if bias is not None else 0.0)
    return math.sqrt(u2)


def term_scales(a: torch.Tensor, b: torch.Tensor) -> list[float]:
    """``U`` of each member ``a[i]·b[i]`` of a stacked batch."""
    p = torch.zeros(a.shape[0], a.shape[1], b.shape[2], dtype=torch.float32, device="cuda")
    rows = measure_batch_rows([(a[i], b[i], p[i], None, i + 1) for i in range(a.shape[0])],
                              h=bytes(32), k=1)
    return [math.sqrt(r[3]) for r in rows.tolist()]


def finish_row(row: Sequence[float], *, q: int, n: int, eps_in: float, eps_acc: float,
               guard: bool = True, biased: bool = False) -> ProductMeasure:
    """The :class:`ProductMeasure` of one product from its row, on the host. ``q`` is the
    checked contraction length (+1 with a bias), ``n`` the rows of ``A``."""
    nu, p_abs1, p_norm, u2, bias_sq, *res = row
    if biased:
        u2 += n * bias_sq
    mp = _measure(nu, p_abs1, tuple(res), p_norm, q, eps_in, eps_acc, math.sqrt(u2))
    return mp if guard else replace(mp, kappa=math.nan)


@dataclass(frozen=True)
class RowArrays:
    """:func:`finish_row`'s fields for ``M`` rows as fp64 arrays (``residuals`` and
    ``normalized`` are ``[M, k]``)."""

    nu: np.ndarray
    p_abs1: np.ndarray
    kappa: np.ndarray
    residuals: np.ndarray
    p_norm: np.ndarray
    unit: np.ndarray
    normalized: np.ndarray
    u: np.ndarray

    def measure(self, i: int) -> ProductMeasure:
        return ProductMeasure(float(self.nu[i]), float(self.p_abs1[i]), float(self.kappa[i]),
                              tuple(self.residuals[i].tolist()), float(self.p_norm[i]),
                              float(self.unit[i]), tuple(self.normalized[i].tolist()),
                              float(self.u[i]))


def finish_row_arrays(rows: np.ndarray, *, q: Sequence[int], n: Sequence[int], eps_in: float,
                      eps_acc: float, guard: bool = True,
                      biased: Sequence[bool] | None = None) -> RowArrays:
    """:func:`finish_row` for every row of ``rows`` (fp64 ``[M, 5 + k]``) at once, with the
    same IEEE operations in the same order on arrays, so every field equals
    :func:`finish_row`'s bit for bit; one array pass instead of a Python loop per product."""
    rows = np.asarray(rows, dtype=np.float64)
    m = rows.shape[0]
    qf = np.asarray(q, dtype=np.float64)
    nf = np.asarray(n, dtype=np.float64)
    nu, p_abs1, p_norm, u2, bias_sq = (rows[:, c] for c in range(5))
    res = rows[:, 5:]
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        if biased is not None:
            u2 = np.where(np.asarray(biased, dtype=bool), u2 + nf * bias_sq, u2)
        u = np.sqrt(u2)
        kappa = np.where(p_abs1 > 0, nu / p_abs1, np.where(nu == 0, 1.0, np.inf))
        if not guard:
            kappa = np.full(m, np.nan)
        zero = p_norm == 0
        # term_ratio: U/‖P‖_F, 1 when both are 0, inf when only ‖P‖_F is (NaN below 0)
        ratio = np.where(zero, np.where(u == 0, 1.0, np.where(u > 0, np.inf, np.nan)),
                         u / p_norm)
        e = math.sqrt(2.0) * eps_in + np.sqrt(qf) * eps_acc * np.maximum(1.0, ratio)
        e = np.where(np.isnan(ratio), np.nan, e)
        unit = np.where(zero, SIGMA_R * np.sqrt(qf) * eps_acc * u, SIGMA_R * e * p_norm)
        normalized = np.where(unit[:, None] > 0, res / unit[:, None],
                              np.where(res == 0, 0.0, np.inf))
    return RowArrays(nu, p_abs1, kappa, res, p_norm, unit, normalized, u)


def finish_rows(rows: np.ndarray, *, q: Sequence[int], n: Sequence[int], eps_in: float,
                eps_acc: float, guard: bool = True,
                biased: Sequence[bool] | None = None) -> list[ProductMeasure]:
    """:func:`finish_row_arrays` as one :class:`ProductMeasure` per row."""
    f = finish_row_arrays(rows, q=q, n=n, eps_in=eps_in, eps_acc=eps_acc, guard=guard,
                          biased=biased)
    cols = (f.nu.tolist(), f.p_abs1.tolist(), f.kappa.tolist(), f.residuals.tolist(),
            f.p_norm.tolist(), f.unit.tolist(), f.normalized.tolist(), f.u.tolist())
    return [ProductMeasure(a, b, kp, tuple(r), pn, un, tuple(nz), uu)
            for a, b, kp, r, pn, un, nz, uu in zip(*cols)]


def band_unit(q: int, eps_in: float, eps_acc: float, p_norm: float, u: float) -> float:
    """``σ_r·e_m·‖P‖_F``; ``σ_r·√q·ε_acc·U`` when ``‖P‖_F = 0``."""
    if p_norm == 0:
        return SIGMA_R * math.sqrt(q) * eps_acc * u
    return SIGMA_R * product_e_m(q, eps_in, eps_acc, p_norm, u) * p_norm


def _measure(nu: float, p_abs1: float, res: tuple[float, ...], p_norm: float, q: int,
             eps_in: float, eps_acc: float, u: float) -> ProductMeasure:
    kappa = nu / p_abs1 if p_abs1 > 0 else (1.0 if nu == 0 else float("inf"))
    unit = band_unit(q, eps_in, eps_acc, p_norm, u)
    normalized = tuple(x / unit if unit > 0 else (0.0 if x == 0 else float("inf")) for x in res)
    return ProductMeasure(nu, p_abs1, kappa, res, p_norm, unit, normalized, u)
