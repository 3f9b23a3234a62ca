"""Sizing formulas for the repetition count ``k`` (reference:
verification/verifier/matmul_check/sizing.py). Pure float math."""

from __future__ import annotations

import math
from dataclasses import dataclass

from verification.parameters import LAMBDA, LOG2_G

Z: float = 8.0
F_TARGET: float = 1.0
C_ANTI: float = math.sqrt(2.0 / 3.0)


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


def b0(f: float, tau: float, e: float, c: float = C_ANTI) -> float:
    return math.log2(f / (tau * e)) + math.log2(1.0 / c)


def bit_budget(lam: float, T: int, M: int, log2G: float) -> float:
    return lam + math.log2(T) + math.log2(M) + log2G


def k_required(N: float, b0_bits: float) -> int:
    if not b0_bits > 0:
        raise ValueError(f"b0 = {b0_bits} bits <= 0: no finite k meets the budget")
    return math.ceil(N / b0_bits)


def f_achieved(c: float, tau: float, e: float, N: float, k: int) -> float:
    return c * tau * e * 2.0 ** (N / k)


@dataclass(frozen=True)
class Sizing:
    q_max: int
    eps_in: float
    eps_acc: float
    e_max: float
    tau: float
    f: float
    c: float
    b0: float
    lam: float
    T: int
    M: int
    log2G: float
    N: float
    k: int
    f_achieved: float
    e_qmax: float = math.nan
    e_cal: float | None = None
    e_cal_at: str | None = None


def size_k(q_max: int, eps_in: float, eps_acc: float, T: int, M: int, *, s_h: float = 1.0,
           z: float = Z, f: float = F_TARGET, c: float = C_ANTI, lam: float = LAMBDA,
           log2G: float = LOG2_G, e_cal: float | None = None,
           e_cal_at: str | None = None) -> Sizing:
    e_q = e_m(q_max, eps_in, eps_acc)
    if e_cal is not None and not math.isfinite(e_cal):
        raise ValueError(f"the largest calibration e_m is {e_cal} ({e_cal_at})")
    e = e_q if e_cal is None else max(e_q, e_cal)
    tau = z * s_h
    bits = b0(f, tau, e, c)
    N = bit_budget(lam, T, M, log2G)
    k = k_required(N, bits)
    return Sizing(q_max=q_max, eps_in=eps_in, eps_acc=eps_acc, e_max=e, tau=tau, f=f, c=c,
                  b0=bits, lam=lam, T=T, M=M, log2G=log2G, N=N, k=k,
                  f_achieved=f_achieved(c, tau, e, N, k), e_qmax=e_q, e_cal=e_cal,
                  e_cal_at=e_cal_at)
