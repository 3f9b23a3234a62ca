"""The twin pass: two products whose A operands are X and Xᵀ (the attention probabilities for
O and dV, δS for dQ and dK, a linear layer's output gradient for dX and G, the logits'
gradient for dF and G_head) measured from one read of X.

Each twin's rows must match the fp64 oracle of the reference's formulas
(freivalds.py:290-321) as any product's do, and the plan that copies Xᵀ to row-major and
measures the two products apart; verdicts must equal the oracle's judgement of the rows.
Tolerances as in test_freivalds_gpu.py: the non-negative sums to 1e-5 relative, bf16
residuals to 1e-4 relative with a floor of two band units.
"""

from __future__ import annotations

import math

import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu
H = bytes(range(32))
BF16, FP32 = 2.0**-8, 2.0**-24
bf = torch.bfloat16


def _twin(rows, cols, w1, w2, seed):
    """X [rows, cols], m₁ = X·B₁ and m₂ = Xᵀ·B₂, products rounded to bf16 from fp32 sums."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g).to(bf)
    b1 = (torch.randn(cols, w1, generator=g) / math.sqrt(cols)).to(bf)
    b2 = (torch.randn(rows, w2, generator=g) / math.sqrt(rows)).to(bf)
    p1 = (x.float() @ b1.float()).to(bf)
    p2 = (x.float().t() @ b2.float()).to(bf)
    return x, b1, b2, p1, p2


def _check(got, a, b, p, r):
    ref = O.measure_row_f64(a.float(), b.float(), p.float(), r)
    for c in range(4):
        assert got[c] == pytest.approx(ref[c], rel=1e-5, abs=1e-30), (c, got[c], ref[c])
    unit = O.finish_row(ref, q=a.shape[1], n=a.shape[0], eps_in=BF16, eps_acc=FP32)["unit"]
    for j, (x, y) in enumerate(zip(got[5:], ref[5:])):
        assert x == pytest.approx(y, rel=1e-4, abs=2 * unit), (j, x, y, unit)
    return ref


def _plan_rows(lib, prods, k):
    plan = lib.fv_plan(prods, k)
    try:
        return plan.twins, plan.rows(H).cpu().tolist()
    finally:
        plan.close()


# (rows, cols): one tile and less than a strip group; several row tiles, the last partial;
# several column tiles, the last partial; the attention members' square shape; a tall one.
SHAPES = [(16, 128), (48, 384), (528, 1152), (1040, 2176), (2048, 2048), (4096, 256)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("k", [1, 2, 3, 4])
def test_twin_rows_match_the_oracle_and_the_separate_plan(lib, shape, k):
    from verification.commitment.native import FvProduct
    rows, cols = shape
    x, b1, b2, p1, p2 = _twin(rows, cols, 40, 72, rows + cols + k)
    xd = x.cuda()
    twin = [FvProduct(xd, b1.cuda(), p1.cuda(), 3), FvProduct(xd.t(), b2.cuda(), p2.cuda(), 8)]
    n_twins, got = _plan_rows(lib, twin, k)
    assert n_twins == 1
    apart = [FvProduct(xd, b1.cuda(), p1.cuda(), 3),
             FvProduct(xd.t().contiguous(), b2.cuda(), p2.cuda(), 8)]
    n_apart, sep = _plan_rows(lib, apart, k)
    assert n_apart == 0
    r1 = O.challenge_matrices(H, [3], k, 40)[0]
    r2 = O.challenge_matrices(H, [8], k, 72)[0]
    _check(got[0], x, b1, p1, r1)
    _check(got[1], x.t(), b2, p2, r2)
    for g_row, s_row in zip(got, sep):
        for c in range(4):
            assert g_row[c] == pytest.approx(s_row[c], rel=1e-5), c


def test_twin_catches_a_forged_entry_in_either_product(lib):
    from verification.commitment.native import FvProduct, verdict_specs
    x, b1, b2, p1, p2 = _twin(1040, 2176, 64, 128, 7)
    p1f, p2f = p1.clone(), p2.clone()
    p1f[1000, 3] += 256.0
    p2f[2100, 100] -= 256.0
    xd = x.cuda()
    prods = [FvProduct(xd, b1.cuda(), p1f.cuda(), 1), FvProduct(xd, b1.cuda(), p1.cuda(), 2),
             FvProduct(xd.t(), b2.cuda(), p2.cuda(), 3),
             FvProduct(xd.t(), b2.cuda(), p2f.cuda(), 4)]
    plan = lib.fv_plan(prods, 4)
    assert plan.twins == 2
    rows = plan.rows(H)
    specs = verdict_specs([2176, 2176, 1040, 1040], [1040, 1040, 2176, 2176], [False] * 4,
                          [1e4] * 4)
    codes, _, first = lib.verdicts(rows, specs, k=4, eps_in=BF16, eps_acc=FP32, tau=8.0)
    got = [tuple(c) for c in codes.cpu().tolist()]
    plan.close()
    host = rows.cpu().tolist()
    for i, (a, b, p, m) in enumerate([(x, b1, p1f, 1), (x, b1, p1, 2), (x.t(), b2, p2, 3),
                                      (x.t(), b2, p2f, 4)]):
        r = O.challenge_matrices(H, [m], 4, b.shape[1])[0]
        ref = _check(host[i], a, b, p, r)
        mp = O.finish_row(ref, q=a.shape[1], n=a.shape[0], eps_in=BF16, eps_acc=FP32)
        assert got[i] == O.judge(mp, tau=8.0, kappa_max=1e4), i
    assert got[0][0] == O.RESIDUAL and got[3][0] == O.RESIDUAL
    assert got[1][0] == got[2][0] == O.ACCEPT and int(first.item()) == 0


def test_twin_with_non_finite_and_fallbacks(lib):
    """A NaN in X reaches both products' rows; a transposed operand the twin pass does not
    take (k = 5, columns not a multiple of 128, or no row-major twin) is copied and measured
    apart, with the same rows."""
    from verification.commitment.native import FvProduct, _twin_mates
    x, b1, b2, p1, p2 = _twin(64, 256, 16, 24, 5)
    xn = x.clone()
    xn[10, 200] = float("nan")
    xd = xn.cuda()
    n_twins, got = _plan_rows(lib, [FvProduct(xd, b1.cuda(), p1.cuda(), 1),
                                    FvProduct(xd.t(), b2.cuda(), p2.cuda(), 2)], 4)
    assert n_twins == 1
    assert all(math.isnan(got[i][0]) and math.isnan(got[i][5]) for i in (0, 1))
    xd = x.cuda()
    prods = [FvProduct(xd, b1.cuda(), p1.cuda(), 1), FvProduct(xd.t(), b2.cuda(), p2.cuda(), 2)]
    assert _twin_mates(prods, 5) == {} and _twin_mates(prods, 4) == {1: 0}
    n5, rows5 = _plan_rows(lib, prods, 5)
    assert n5 == 0
    _check(rows5[1], x.t(), b2, p2, O.challenge_matrices(H, [2], 5, 24)[0])
    y, c1, c2, q1, q2 = _twin(64, 200, 16, 24, 6)  # 200 columns: not a multiple of 128
    yd = y.cuda()
    odd = [FvProduct(yd, c1.cuda(), q1.cuda(), 1), FvProduct(yd.t(), c2.cuda(), q2.cuda(), 2)]
    assert _twin_mates(odd, 4) == {}
    n_odd, rows_odd = _plan_rows(lib, odd, 4)
    assert n_odd == 0
    _check(rows_odd[1], y.t(), c2, q2, O.challenge_matrices(H, [2], 4, 24)[0])
    alone = [FvProduct(xd.t(), b2.cuda(), p2.cuda(), 2)]  # no row-major twin in the plan
    assert _twin_mates(alone, 4) == {}
    assert _plan_rows(lib, alone, 4)[0] == 0


def test_twins_beside_other_products(lib):
    """Two twins over different X, a third product reading one X row-major again, and
    unrelated fp32 and bf16 products in one plan: every row as the oracle's."""
    from verification.commitment.native import FvProduct
    xa, a1, a2, pa1, pa2 = _twin(512, 1024, 128, 128, 21)
    xb, c1, c2, pb1, pb2 = _twin(2048, 384, 48, 2048, 22)
    d = (torch.randn(1024, 64) / 32).to(bf)
    pd = (xa.float() @ d.float()).to(bf)
    e = torch.randn(96, 80)
    f = torch.randn(80, 33) / 9
    pe = e @ f
    dev = [t.cuda() for t in (xa, xb)]
    prods = [FvProduct(e.cuda(), f.cuda(), pe.cuda(), 1),
             FvProduct(dev[0], a1.cuda(), pa1.cuda(), 2),
             FvProduct(dev[1].t(), c2.cuda(), pb2.cuda(), 3),
             FvProduct(dev[0], d.cuda(), pd.cuda(), 4),
             FvProduct(dev[1], c1.cuda(), pb1.cuda(), 5),
             FvProduct(dev[0].t(), a2.cuda(), pa2.cuda(), 6)]
    n_twins, got = _plan_rows(lib, prods, 4)
    assert n_twins == 2
    want = [(e, f, pe, 1), (xa, a1, pa1, 2), (xb.t(), c2, pb2, 3), (xa, d, pd, 4),
            (xb, c1, pb1, 5), (xa.t(), a2, pa2, 6)]
    for i, (a, b, p, m) in enumerate(want):
        r = O.challenge_matrices(H, [m], 4, b.shape[1])[0]
        if a.dtype == torch.float32:
            ref = O.measure_row_f64(a, b, p, r)
            for c in range(4):
                assert got[i][c] == pytest.approx(ref[c], rel=1e-5), (i, c)
        else:
            _check(got[i], a, b, p, r)
