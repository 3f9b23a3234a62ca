"""Parity of the gfx950 challenge, Freivalds and verdict kernels with the CPU oracle.

Tolerances, per column:
- challenges: bit for bit;
- ν, ‖|P|·1‖, ‖P‖_F, ΣA²(B²1), ‖b‖² (sums of non-negative terms): relative 1e-5;
- residuals dominated by a planted error, and residuals of bf16 products (dominated by the
  committed leaf's own rounding): relative 1e-4;
- honest fp32 residuals (pure rounding noise): within 2 band units of the fp64 value;
- verdicts from the same rows: bit for bit (codes and the finished κ, unit, U).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
H = bytes(range(32))
FP32, BF16 = 2.0**-24, 2.0**-8


# ---- challenges ----------------------------------------------------------------------------

@pytest.mark.parametrize("width", [1, 5, 16, 17, 256, 257, 1000, 4096])
@pytest.mark.parametrize("k", [1, 3, 16, 20])
def test_challenges_bit_exact(lib, width, k):
    ms = [1, 2, 77, 2**32 - 1]
    got = lib.challenge_matrices(H, ms, k, width).cpu()
    want = O.challenge_matrices(H, ms, k, width)
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))


def test_challenge_known_answer(lib):
    r = lib.challenge_matrices(bytes(32), [1], 1, 4)[0, :, 0].cpu()
    assert r.tolist() == [n / 2**24 for n in (9704253, 8138245, 496685, -7670651)]
    assert [f"{v:08x}" for v in r.numpy().view(np.uint32)] == \
        ["3f14133d", "3ef85c0a", "3cf285a0", "beea16f6"]


def test_challenge_api(lib):
    from verification.verifier.matmul_check.challenges import (challenge_matrix,
                                                               challenge_vector, encode_label)
    assert encode_label(1, 1) == b"\x10\x00\x00\x00\x01\x01"
    R = challenge_matrix(H, 11, 7, 257).cpu()
    for j in range(1, 8):
        assert torch.equal(R[:, j - 1], challenge_vector(H, 11, j, 257).cpu())
    assert torch.equal(R, O.challenge_matrix_xof(H, 11, 7, 257))
    with pytest.raises(ValueError):
        challenge_matrix(H, 0, 1, 4)
    with pytest.raises(ValueError):
        challenge_matrix(H, 1, 256, 4)
    with pytest.raises(ValueError):
        challenge_matrix(b"short", 1, 1, 4)


# ---- Freivalds rows ------------------------------------------------------------------------

def _operands(n, q, w, seed, dtype, bias=False, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    a = (torch.randn(n, q, generator=g) * scale).to(dtype)
    b = (torch.randn(q, w, generator=g) / math.sqrt(q)).to(dtype)
    bv = torch.randn(w, generator=g).to(dtype).float() if bias else None
    p = a.float() @ b.float()
    if bv is not None:
        p = p + bv
    return a, b, p.to(dtype), bv


def _check_row(got, a, b, p, r, bias, dtype, planted=False):
    want = O.measure_product_row(a.float(), b.float(), p.float(), r, bias)
    ref64 = O.measure_row_f64(a.float(), b.float(), p.float(), r, bias)
    for c in range(5):
        if math.isnan(want[c]):
            assert math.isnan(got[c])
        else:
            assert got[c] == pytest.approx(want[c], rel=1e-5, abs=1e-30), (c, got[c], want[c])
    q = a.shape[1] + (bias is not None)
    mp = O.finish_row(ref64, q=q, n=a.shape[0], eps_in=FP32 if dtype == torch.float32 else BF16,
                      eps_acc=FP32, biased=bias is not None)
    for j, (x, y) in enumerate(zip(got[5:], ref64[5:])):
        if planted or dtype == torch.bfloat16:
            assert x == pytest.approx(y, rel=1e-4, abs=2 * mp["unit"]), (j, x, y)
        else:
            assert abs(x - y) <= 2 * mp["unit"], (j, x, y, mp["unit"])


# (n, q, w): aligned and unaligned rows, partial pipeline stages, and q or w past one
# 4096-column chunk (several chunks reduced in order).
SHAPES = [(64, 32, 48), (100, 77, 130), (13, 8, 12), (256, 576, 192), (1, 5, 3), (65, 33, 17),
          (70, 4500, 40), (33, 48, 8300)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", SHAPES)
# k spans one to five 16-slot column groups (bf16: 5 columns a group; fp32: 16).
@pytest.mark.parametrize("k", [1, 4, 12, 16, 20, 24])
def test_rows_match_oracle(lib, dtype, shape, k):
    from verification.verifier.matmul_check.freivalds import measure_batch_rows
    n, q, w = shape
    a, b, p, _ = _operands(n, q, w, 11 * n + q + w + k, dtype)
    rows = measure_batch_rows([(a, b, p, None, 5)], h=H, k=k).cpu()
    r = O.challenge_matrices(H, [5], k, w)[0]
    _check_row(rows[0].tolist(), a, b, p, r, None, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_biased_rows(lib, dtype):
    from verification.verifier.matmul_check.freivalds import measure_batch_rows
    a, b, p, bias = _operands(96, 64, 80, 3, dtype, bias=True)
    rows = measure_batch_rows([(a, b, p, bias, 9)], h=H, k=4).cpu()
    r = O.challenge_matrices(H, [9], 4, 80)[0]
    _check_row(rows[0].tolist(), a, b, p, r, bias, dtype)


def test_many_products_one_plan(lib):
    """A batch mixing shapes, dtypes, biases and member stacks, as check 5 sees a step."""
    from verification.verifier.matmul_check.freivalds import measure_batch_rows
    items, ref = [], []
    for i, (shape, dtype, biased) in enumerate([((128, 96, 64), torch.bfloat16, True),
                                                ((64, 128, 96), torch.bfloat16, False),
                                                ((50, 40, 30), torch.float32, False),
                                                ((256, 64, 256), torch.bfloat16, False)]):
        a, b, p, bias = _operands(*shape, 40 + i, dtype, bias=biased)
        items.append((a, b, p, bias, 100 + i))
        ref.append((a, b, p, bias, dtype))
    rows = measure_batch_rows(items, h=H, k=3).cpu()
    for i, (a, b, p, bias, dtype) in enumerate(ref):
        r = O.challenge_matrices(H, [100 + i], 3, p.shape[1])[0]
        _check_row(rows[i].tolist(), a, b, p, r, bias, dtype)


def test_members_match_oracle(lib):
    from verification.verifier.matmul_check.freivalds import measure_products_rows
    g = torch.Generator().manual_seed(5)
    a = torch.randn(6, 64, 32, generator=g).to(torch.bfloat16)
    b = torch.randn(6, 32, 64, generator=g).to(torch.bfloat16)
    p = torch.bmm(a.float(), b.float()).to(torch.bfloat16)
    ms = [10, 12, 14, 16, 18, 20]
    rows = measure_products_rows(a.to(DEV), b.to(DEV), p.to(DEV), h=H, ms=ms, k=2).cpu()
    R = O.challenge_matrices(H, ms, 2, 64)
    want = O.measure_products_rows(a, b, p, R)
    for i in range(6):
        assert rows[i, :4].tolist() == pytest.approx(want[i][:4], rel=1e-5)
        assert rows[i, 5:].tolist() == pytest.approx(want[i][5:], rel=1e-4)


def test_planted_error_is_measured(lib):
    from verification.verifier.matmul_check.freivalds import measure_batch_rows
    a, b, p, _ = _operands(128, 64, 96, 8, torch.float32)
    p2 = p.clone()
    p2[17, 33] += 0.05
    rows = measure_batch_rows([(a, b, p2, None, 3)], h=H, k=8).cpu()
    r = O.challenge_matrices(H, [3], 8, 96)[0]
    _check_row(rows[0].tolist(), a, b, p2, r, None, torch.float32, planted=True)
    # the residual of challenge j is |0.05 · r_j[33]| to fp32 accuracy
    for j in range(8):
        assert rows[0, 5 + j].item() == pytest.approx(abs(0.05 * r[33, j].item()), rel=1e-3)


def test_large_entries_zero_product_and_nan(lib):
    from verification.verifier.matmul_check.freivalds import measure_batch_rows
    a, b, p, _ = _operands(32, 16, 24, 1, torch.float32)
    big = p.clone()
    big[0, 0] = 3e19
    big[1, 1] = -3e19
    zero = torch.zeros_like(p)
    nan = p.clone()
    nan[2, 3] = float("nan")
    rows = measure_batch_rows([(a, b, big, None, 1), (a, b, zero, None, 2),
                               (a, b, nan, None, 3), (a, b, p, None, 4)], h=H, k=2).cpu()
    assert math.isfinite(rows[0, 2].item())
    assert rows[0, 2].item() == pytest.approx(math.sqrt(2) * 3e19, rel=1e-6)
    assert rows[1, 2].item() == 0.0 and rows[1, 1].item() == 0.0
    assert math.isnan(rows[2, 2].item()) and math.isnan(rows[2, 5].item())
    assert all(math.isfinite(x) for x in rows[3].tolist())  # NaN stays inside its product


def test_guard_off_gives_nan_guard_columns(lib):
    from verification.verifier.matmul_check.freivalds import measure_batch_rows
    a, b, p, _ = _operands(32, 16, 24, 2, torch.float32)
    on = measure_batch_rows([(a, b, p, None, 1)], h=H, k=2).cpu()[0]
    off = measure_batch_rows([(a, b, p, None, 1)], h=H, k=2, guard=False).cpu()[0]
    assert math.isnan(off[0]) and math.isnan(off[1])
    assert torch.equal(on[2:], off[2:])


def test_strided_rows_and_views(lib):
    from verification.verifier.matmul_check.freivalds import measure_batch_rows
    big_a = torch.randn(64, 50).to(torch.bfloat16)
    big_b = torch.randn(40, 70).to(torch.bfloat16)
    a, b = big_a[:, 3:43], big_b[:, 5:61]   # row strides 50 and 70: unaligned rows
    p = (a.float() @ b.float()).to(torch.bfloat16)
    rows = measure_batch_rows([(a.to(DEV), b.to(DEV), p.to(DEV), None, 7)], h=H, k=4).cpu()
    r = O.challenge_matrices(H, [7], 4, 56)[0]
    _check_row(rows[0].tolist(), a, b, p, r, None, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_transposed_operands(lib, dtype):
    """Captured operands come as transposed views (a linear layer's ``B = W.t()``, a weight
    gradient's ``A = δYᵀ``): the rows equal those of row-major copies bit for bit."""
    from verification.commitment import native
    a, b, p, bv = _operands(96, 130, 70, 5, dtype, bias=True)
    a_t = a.t().contiguous().to(DEV).t()   # [n, q] with strides (1, n)
    b_t = b.t().contiguous().to(DEV).t()   # [q, w] with strides (1, q)
    assert a_t.stride() == (1, 96) and b_t.stride() == (1, 130)

    def rows(x, y):
        plan = lib.fv_plan([native.FvProduct(x, y, p.to(DEV), 9, bv.to(DEV))], 4, True)
        try:
            return plan.rows(H).cpu()
        finally:
            plan.close()

    got = rows(a_t, b_t)
    assert torch.equal(got, rows(a.to(DEV), b.to(DEV)))
    r = O.challenge_matrices(H, [9], 4, 70)[0]
    _check_row(got[0].tolist(), a, b, p, r, bv, dtype)


def test_plan_challenges_equal_oracle(lib):
    from verification.commitment import native
    a, b, p, _ = _operands(32, 16, 40, 2, torch.bfloat16)
    a2, b2, p2, _ = _operands(16, 8, 24, 3, torch.float32)
    plan = lib.fv_plan([native.FvProduct(a.to(DEV), b.to(DEV), p.to(DEV), 3),
                        native.FvProduct(a2.to(DEV), b2.to(DEV), p2.to(DEV), 9)], 5)
    plan.rows(H)
    R = plan.challenges()
    assert torch.equal(R[0].cpu(), O.challenge_matrices(H, [3], 5, 40)[0])
    assert torch.equal(R[1].cpu(), O.challenge_matrices(H, [9], 5, 24)[0])


# ---- verdicts ------------------------------------------------------------------------------

def _edge_rows(k):
    rng = np.random.default_rng(0)
    rows = []
    for _ in range(300):
        nu, p1, pn = (float(x) for x in rng.lognormal(0, 2, 3))
        u2 = float(rng.lognormal(0, 3))
        res = [float(x) for x in rng.lognormal(-12, 3, k)]
        rows.append([nu, p1, pn, u2, float(rng.lognormal(-2, 1)), *res])
    special = [0.0, -0.0, float("inf"), float("nan"), 1e-300, 1e300, 5e-324]
    for i, v in enumerate(special):
        for col in range(5 + k):
            r = list(rows[i])
            r[col] = v
            rows.append(r)
    rows.append([0.0, 0.0, 0.0, 0.0, 0.0] + [0.0] * k)
    rows.append([1.0, 0.0, 0.0, 4.0, 0.0] + [1e-9] * k)
    return rows


@pytest.mark.parametrize("guard", [True, False])
@pytest.mark.parametrize("biased", [False, True])
def test_verdicts_bit_exact_with_python(lib, guard, biased):
    from verification.commitment import native
    k = 3
    rows = _edge_rows(k)
    n = len(rows)
    rng = np.random.default_rng(1)
    qs = [int(x) for x in rng.integers(2, 200_000, n)]
    ns = [int(x) for x in rng.integers(1, 10_000, n)]
    kap = [float(x) for x in rng.choice([10.0, 1e4, 3.5], n)]
    specs = native.verdict_specs(qs, ns, [biased] * n, kap)
    dr = torch.tensor(rows, dtype=torch.float64, device=DEV)
    codes, fin, first = lib.verdicts(dr, specs, k=k, eps_in=BF16, eps_acc=FP32, tau=8.0,
                                     guard=guard, finished=True)
    codes, fin = codes.cpu().tolist(), fin.cpu().tolist()
    first_want = n
    for i, row in enumerate(rows):
        mp = O.finish_row(row, q=qs[i], n=ns[i], eps_in=BF16, eps_acc=FP32, biased=biased)
        want = O.judge(mp, tau=8.0, kappa_max=kap[i], guard=guard)
        assert tuple(codes[i]) == want, (i, row)
        for got, ref in zip(fin[i], [mp["kappa"] if guard else float("nan"), mp["unit"], mp["u"]]):
            assert (math.isnan(got) and math.isnan(ref)) or got == ref, (i, got, ref)
        if want[0] != 0:
            first_want = min(first_want, i)
    assert int(first.item()) == first_want


@pytest.mark.parametrize("k", [4, 7, 16])
def test_grid_limited_passes_take_tiles_from_a_queue(lib, k):
    """Row passes limited to fewer blocks than they have tiles take their tiles from a queue
    that each launch resets, each lane loading its own V, where a block per tile shares each
    stage's V through LDS: two runs in a row give the rows of the plan with a block per tile
    bit for bit, for bf16 and fp32 operands and a bias, with one, two and four 16-column
    groups of V (k = 4, 7, 16)."""
    from verification.commitment import native
    items = []
    for i, (shape, dtype, biased) in enumerate([((1024, 2048, 640), torch.bfloat16, True),
                                                ((777, 4500, 300), torch.bfloat16, False),
                                                ((300, 1100, 200), torch.float32, False),
                                                ((2048, 256, 1536), torch.bfloat16, False)]):
        a, b, p, bias = _operands(*shape, 70 + i, dtype, bias=biased)
        items.append(native.FvProduct(a.cuda(), b.cuda(), p.cuda(), 200 + i,
                                      None if bias is None else bias.cuda()))
    want = lib.fv_plan(items, k).rows(H)
    plan = lib.fv_plan(items, k)
    for stage, blocks in ((1, 3), (3, 5), (4, 7)):
        plan.set_grid(stage, blocks)
    for _ in range(2):
        got = plan.rows(H)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int64), want.view(torch.int64))


@pytest.mark.parametrize("k", [4, 7, 16])
def test_grid_limited_passes_short_chunks(lib, k):
    """Grid-limited row passes over chunks of a few whole stages (bf16: 128 columns a stage,
    fp32: 64), where the pairs of stages whose next stage is whole run in their own loop and
    the last stages in the general one: three, four and five whole stages, with and without a
    last partial stage that ends on a K-step (416 = 3 x 128 + 32 columns) or inside one
    (424); rows bit for bit those of a block per tile."""
    from verification.commitment import native
    items = []
    for i, (shape, dtype) in enumerate([((200, 384, 96), torch.bfloat16),
                                        ((130, 512, 64), torch.bfloat16),
                                        ((333, 640, 80), torch.bfloat16),
                                        ((150, 416, 72), torch.bfloat16),
                                        ((90, 424, 40), torch.bfloat16),
                                        ((120, 320, 48), torch.float32)]):
        a, b, p, _ = _operands(*shape, 110 + i, dtype)
        items.append(native.FvProduct(a.cuda(), b.cuda(), p.cuda(), 400 + i))
    want = lib.fv_plan(items, k).rows(H)
    plan = lib.fv_plan(items, k)
    for stage, blocks in ((1, 3), (3, 5), (4, 7)):
        plan.set_grid(stage, blocks)
    for _ in range(2):
        got = plan.rows(H)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int64), want.view(torch.int64))


def test_queues_with_fewer_tiles_than_xcds(lib):
    """The tiles are split into one queue per XCD; with fewer tiles than queues some ranges
    are empty, and a grid of 2 blocks must still drain every range (from whichever XCD the
    blocks run on): rows bit for bit those of a block per tile."""
    from verification.commitment import native
    items = []
    for i, (shape, dtype) in enumerate([((100, 96, 80), torch.bfloat16),
                                        ((64, 200, 48), torch.float32),
                                        ((130, 64, 40), torch.bfloat16)]):
        a, b, p, _ = _operands(*shape, 90 + i, dtype)
        items.append(native.FvProduct(a.cuda(), b.cuda(), p.cuda(), 300 + i))
    want = lib.fv_plan(items, 4).rows(H)
    plan = lib.fv_plan(items, 4)
    for stage in (1, 3, 4):
        plan.set_grid(stage, 2)
    for _ in range(2):
        got = plan.rows(H)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int64), want.view(torch.int64))
