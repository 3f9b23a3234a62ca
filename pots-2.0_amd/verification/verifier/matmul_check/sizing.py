"""The honest error model behind check 5's band unit (reference:
verification/verifier/matmul_check/sizing.py:16-43, F18): ``e_m``, its term ratio, and ``Z``,
the provisional band's multiple. The sizing of ``k`` is not part of this build. Pure float
math."""

from __future__ import annotations

import math

Z: float = 8.0


def e_m(q: int, eps_in: float, eps_acc: float, u_ratio: float = 1.0) -> float:
    """Honest relative error ``√2·ε_in + √q·ε_acc·max(1, U/‖P‖_F)``; NaN ratio gives NaN."""
    if math.isnan(u_ratio):
        return math.nan
    return math.sqrt(2.0) * eps_in + math.sqrt(q) * eps_acc * max(1.0, u_ratio)


def term_ratio(p_norm: float, u: float) -> float:
    """``U/‖P‖_F``: inf when only ``‖P‖_F`` is 0 and ``U > 0``, 1 when both are 0."""
    if p_norm == 0 and u == 0:
        return 1.0
    if p_norm == 0:
        return math.inf if u > 0 else math.nan
    return u / p_norm


def product_e_m(q: int, eps_in: float, eps_acc: float, p_norm: float, u: float) -> float:
    return e_m(q, eps_in, eps_acc, term_ratio(p_norm, u))
