"""Host-side logic of the check layer: rejections, the error guard, committed leaves, the
in-memory store and check 5's judging messages (no GPU needed).

The judging tests feed hand-made ProductMeasure values to the judge and compare its
Rejection with the reference's rules and detail strings
(verification/verifier/checks.py:926-956).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from verification.computation.interface import ProductKind, ProductSpec
from verification.transcript.errors import LeafShapeError, StoreMutationError
from verification.transcript.store import InMemoryStore
from verification.verifier.bands import Bands
from verification.verifier.checks import DEFAULT_ORDER, _judge_product, protocol_id
from verification.verifier.context import (CommittedLeaves, Rejection, StepContext, _checked,
                                           _guard, _is_digest)
from verification.verifier.matmul_check.freivalds import ProductMeasure, finish_row


class _C:
    """Enough of a computation for the judge: its product classes."""

    def product_class(self, spec):
        return f"{spec.kind.value}:{spec.name}"


SPEC = ProductSpec(m=7, name="Y_q[0]", kind=ProductKind.FORWARD, a_shape=(4, 8), b_shape=(8, 3))


def _ctx(**kw):
    base = dict(step=3, indices=(), h_D=b"", n_records=0, prev_w_hashes=(), chain_check_id="7",
                k=2, eps_in=2.0**-8, eps_acc=2.0**-24, eps_w=2.0**-24)
    base.update(kw)
    return StepContext(**base)


def _mp(nu=1.0, p_abs1=1.0, res=(0.0, 0.0), p_norm=1.0, unit=1e-3, u=1.0):
    kappa = nu / p_abs1 if p_abs1 > 0 else (1.0 if nu == 0 else math.inf)
    normalized = tuple(x / unit for x in res)
    return ProductMeasure(nu, p_abs1, kappa, tuple(res), p_norm, unit, normalized, u)


def test_slot_order_and_ids():
    assert DEFAULT_ORDER == ("7", "2", "6a", "5", "6b", "2.root")
    assert protocol_id("2.root") == "2" and protocol_id("5") == "5"


def test_guard_maps_prover_errors_to_malformed():
    ctx = _ctx()

    @_checked
    def check():
        with _guard(ctx, "2"):
            raise LeafShapeError("leaf 4 W_t[x]: shape (2, 2), declared (2, 3)")

    rej = check()
    assert rej == Rejection(3, "2", "malformed prover data: LeafShapeError: leaf 4 W_t[x]: "
                                    "shape (2, 2), declared (2, 3)", "malformed")

    @_checked
    def bug():
        with _guard(ctx, "2"):
            raise RuntimeError("a verifier bug propagates")

    with pytest.raises(RuntimeError):
        bug()


def test_committed_leaves_detect_in_place_writes():
    leaves = CommittedLeaves()
    t = torch.zeros(3)
    leaves.add(t)
    assert leaves.leaf(0) is t and not leaves.changed(0)
    t.add_(1)
    assert leaves.changed(0)
    with pytest.raises(StoreMutationError):
        leaves.leaf(0)
    with pytest.raises(RuntimeError):
        leaves.leaf(5)


def test_in_memory_store_versions_and_root():
    t = torch.ones(4)
    s = InMemoryStore([t], claimed_root=b"\x01" * 32)
    assert s.root == b"\x01" * 32 and s.leaf(0) is t
    t.mul_(2)
    with pytest.raises(StoreMutationError):
        s.leaf(0)
    with pytest.raises(IndexError):
        s.leaf(1)
    with pytest.raises(LookupError):
        s.path(0)
    assert _is_digest(b"\0" * 32) and not _is_digest(b"\0" * 31) and not _is_digest("x" * 32)


def test_judge_accepts_and_records():
    ctx = _ctx()
    assert _judge_product(_C(), SPEC, _mp(res=(1e-3, 2e-3)), ctx, Bands.provisional()) is None
    (st,) = ctx.stats.products
    assert (st.m, st.name, st.cls, st.kappa, st.normalized) == \
        (7, "Y_q[0]", "forward:Y_q[0]", 1.0, (1.0, 2.0))


def test_judge_residual_message():
    ctx = _ctx()
    rej = _judge_product(_C(), SPEC, _mp(res=(1e-3, 9e-3)), ctx, Bands.provisional())
    assert rej == Rejection(3, "5", "P_7 (Y_q[0]), challenge j=2: normalized residual 9 > τ = 8")


def test_judge_cancellation_message():
    ctx = _ctx()
    bands = Bands(tau=8.0, kappa_max=10.0)
    rej = _judge_product(_C(), SPEC, _mp(nu=50.0, p_abs1=2.0), ctx, bands)
    assert rej == Rejection(3, "5", "P_7 (Y_q[0]): cancellation factor κ = 25 > κ_max = 10 "
                                    "[forward:Y_q[0]]")
    # with the guard off, test 1 is skipped and ν, ‖|P|·1‖ may be NaN
    ctx = _ctx(kappa_guard=False)
    assert _judge_product(_C(), SPEC, _mp(nu=math.nan, p_abs1=math.nan), ctx, bands) is None


def test_judge_non_finite_message_lists_every_bad_value():
    ctx = _ctx()
    rej = _judge_product(_C(), SPEC, _mp(nu=math.inf, res=(math.nan, 0.0)), ctx,
                         Bands.provisional())
    assert rej == Rejection(3, "5", "P_7 (Y_q[0]): non-finite ν, residual j=1")
    # calibration mode records and never judges, but non-finite still rejects
    ctx = _ctx(judge=False)
    assert _judge_product(_C(), SPEC, _mp(res=(1.0, 1.0)), ctx, Bands.provisional()) is None
    assert _judge_product(_C(), SPEC, _mp(u=math.nan), ctx, Bands.provisional()) is not None


def test_nan_never_passes_a_band():
    """A NaN residual that is not caught as non-finite would pass ``x > bound``; the judge
    writes every comparison as ``not (x <= bound)``."""
    ctx = _ctx()
    mp = finish_row([1.0, 1.0, 1.0, 1.0, 0.0, 0.0, 1e30], q=8, n=4, eps_in=2.0**-8,
                    eps_acc=2.0**-24)
    rej = _judge_product(_C(), SPEC, mp, ctx, Bands.provisional())
    assert rej is not None and rej.check_id == "5" and "challenge j=2" in rej.detail


def test_finish_rows_equals_finish_row_bit_for_bit():
    """Check 5 finishes every row at once; each field must equal the per-row closed form,
    including zeros of either sign, NaN, infinities and the biased and unguarded cases."""
    import random

    import numpy as np

    from verification.verifier.matmul_check.freivalds import finish_row, finish_rows
    rng = random.Random(0)
    specials = [0.0, -0.0, 1e-300, 1e300, math.inf, math.nan, 1.0, 3.5e-8]

    def val():
        if rng.random() < 0.3:
            return rng.choice(specials)
        return rng.uniform(0, 10) * 10 ** rng.randint(-12, 6)

    def same(a, b):
        return (math.isnan(a) and math.isnan(b)) or \
            (a == b and math.copysign(1, a) == math.copysign(1, b))

    for k in (1, 4):
        rows = [[val() for _ in range(5 + k)] for _ in range(600)]
        q = [rng.randint(2, 20000) for _ in rows]
        n = [rng.randint(1, 9000) for _ in rows]
        biased = [rng.random() < 0.3 for _ in rows]
        for guard in (True, False):
            got = finish_rows(np.array(rows), q=q, n=n, eps_in=2.0**-8, eps_acc=2.0**-24,
                              guard=guard, biased=biased)
            for r, qq, nn, b, g in zip(rows, q, n, biased, got):
                w = finish_row(r, q=qq, n=nn, eps_in=2.0**-8, eps_acc=2.0**-24, guard=guard,
                               biased=b)
                for f in ("nu", "p_abs1", "kappa", "p_norm", "unit", "u"):
                    assert same(getattr(w, f), getattr(g, f)), (f, r, qq, nn, b)
                assert all(same(x, y) for x, y in zip(w.residuals, g.residuals))
                assert all(same(x, y) for x, y in zip(w.normalized, g.normalized))


def _tiny_decoder():
    from verification.computation.instances.decoder import DecoderComputation
    return DecoderComputation(L=1, d=16, d_f=32, n_h=2, n_kv=1, n_v=40, n_s=1, n=8)


class _RaisingReplay:
    """Operands from a table; product ``bad`` fails to serve with ``error``."""

    def __init__(self, table, bad, error):
        self.table, self.bad, self.error = table, bad, error

    def operands(self, m):
        if m == self.bad:
            raise self.error
        return self.table[m]


def _ctx_after_check_2(c, leaves, **kw):
    ctx = _ctx(**kw)
    committed = CommittedLeaves()
    for obj in leaves:
        committed.add(obj)
    ctx.state.claimed_root, ctx.state.leaves = bytes(32), committed
    return ctx


def _leaves(c):
    from setup.records import Record
    out = [Record(torch.zeros(c.n, dtype=torch.int32), torch.zeros(c.n, dtype=torch.int32),
                  torch.ones(c.n, dtype=torch.int32))]
    out += [torch.zeros(c.weight_shapes[n]) for n in c.weight_names]
    out += [torch.zeros(s.p_shape, dtype=c.product_dtype) for s in c.products]
    out += [torch.zeros(c.weight_shapes[n]) for n in c.weight_names]
    return out


def test_check_5_serving_error_at_the_first_product_is_malformed():
    """A prover-data error while serving product 1 (nothing measured before it) is check 5's
    malformed rejection, returned, not raised (reference checks.py:574,613-650)."""
    from verification.transcript.errors import TranscriptFormatError
    from verification.verifier.checks import check_5_matmuls
    c = _tiny_decoder()
    leaves = _leaves(c)
    c.use_operands(_RaisingReplay({}, 1, TranscriptFormatError("operand file truncated")))
    ctx = _ctx_after_check_2(c, leaves)
    rej = check_5_matmuls(None, c, ctx, Bands.provisional())
    assert rej == Rejection(3, "5", "malformed prover data: TranscriptFormatError: operand "
                                    "file truncated", "malformed")
    assert ctx.state.run_rest_error is None


def test_check_5_leaf_mutated_after_check_2_is_malformed():
    from verification.verifier.checks import check_5_matmuls
    c = _tiny_decoder()
    leaves = _leaves(c)
    table = {s.m: (torch.zeros(s.a_shape), torch.zeros(s.b_shape)) for s in c.products}
    c.use_operands(_RaisingReplay(table, None, None))
    ctx = _ctx_after_check_2(c, leaves)
    leaves[c.product_index(1)].add_(1)  # after check 2 hashed it
    rej = check_5_matmuls(None, c, ctx, Bands.provisional())
    assert rej is not None and (rej.check_id, rej.kind) == ("5", "malformed")
    assert rej.detail.startswith("malformed prover data: StoreMutationError: leaf "
                                 f"{c.product_index(1)} changed in place")


def test_check_5_refuses_untrusted_prover_operands():
    from verification.prover.synthetic import CapturedReplay
    from verification.verifier.checks import check_5_matmuls
    c = _tiny_decoder()
    c.use_operands(CapturedReplay({}))
    with pytest.raises(RuntimeError, match="trust_prover_operands"):
        check_5_matmuls(None, c, _ctx_after_check_2(c, _leaves(c)), Bands.provisional())


def test_verifier_constructor_refuses_what_the_reference_refuses():
    from verification.prover.synthetic import CapturedReplay
    from verification.verifier.driver import Verifier
    c = _tiny_decoder()
    w0 = {n: torch.zeros(c.weight_shapes[n]) for n in c.weight_names}
    base = dict(h_D=bytes(32), n_records=4, k=2, n_steps=3, bands=Bands.provisional(),
                seed=0, w0=w0, allow_provisional=True)

    def refused(match, **kw):
        with pytest.raises(ValueError, match=match):
            Verifier(c, **{**base, **kw})

    refused("exactly one of w0 and w0_hashes", w0_hashes=[bytes(32)] * c.n_w)
    refused("h_D must be a 32-byte digest", h_D=b"x")
    refused("k must be in 1..255", k=0)
    refused("n_steps", n_steps=0)
    refused("bands are required", bands=None)
    refused("allow_provisional", allow_provisional=False)
    refused("κ guard", calibrate=True, kappa_guard=False)
    refused("match no product", bands=Bands(tau=8.0, kappa_max=1e4,
                                            kappa_classes={"no such class": 2.0}))
    c.use_operands(CapturedReplay({}))
    refused("trust_prover_operands")
    v = Verifier(c, **base, trust_prover_operands=True)
    with pytest.raises(RuntimeError, match="start_run"):
        v.verify_step(1, None)
    assert v.band_source == "provisional"


@pytest.mark.parametrize("guard", [True, False])
@pytest.mark.parametrize("judge", [True, False])
@pytest.mark.parametrize("seed", range(6))
def test_array_judge_stops_where_the_per_product_judge_does(guard, judge, seed):
    """Check 5 finds the first rejected product with array tests; on rows with NaN, inf,
    zero norms, κ at and over its band and residuals at and over τ·unit, it must stop at the
    product a per-product ``finish_row`` + ``_judge_product`` loop stops at, record the same
    statistics before it, and word the same rejection."""
    from verification.verifier.checks import _first_rejected, _judge_product, _product_table
    from verification.verifier.matmul_check.freivalds import finish_row, finish_row_arrays
    c = _tiny_decoder()
    bands = Bands.provisional()
    classes, qs, ns, biased = _product_table(c)
    kmax = np.array([bands.kappa_for(cls) for cls in classes])
    g = np.random.default_rng(seed)
    M, k = c.M, 2
    rows = np.abs(g.normal(size=(M, 5 + k)))
    rows[:, 5:] *= 1e-12
    specials = [np.nan, np.inf, 0.0, 1e300]
    for _ in range(3):  # a few rows with special entries at random places
        i, j = g.integers(M), g.integers(5 + k)
        rows[i, j] = specials[g.integers(len(specials))]
    i = g.integers(M)
    rows[i, 1] = rows[i, 0] / kmax[i] * (1 - 1e-12)  # κ just over its band
    ctx = _ctx(k=k, judge=judge, kappa_guard=guard)
    f = finish_row_arrays(rows, q=qs, n=ns, eps_in=ctx.eps_in, eps_acc=ctx.eps_acc,
                          guard=guard, biased=biased)
    i = int(g.integers(M))
    rows[i, 5] = bands.tau * f.unit[i] * (1 + 1e-9)  # a residual just over τ·unit
    f = finish_row_arrays(rows, q=qs, n=ns, eps_in=ctx.eps_in, eps_acc=ctx.eps_acc,
                          guard=guard, biased=biased)
    stop = _first_rejected(f, kmax, ctx, bands)
    ref_ctx = _ctx(k=k, judge=judge, kappa_guard=guard)
    want, ref_rej = M, None
    for m, spec in enumerate(c.products):
        mp = finish_row(rows[m].tolist(), q=spec.q, n=spec.a_shape[0], eps_in=ctx.eps_in,
                        eps_acc=ctx.eps_acc, guard=guard, biased=bool(biased[m]))
        ref_rej = _judge_product(c, spec, mp, ref_ctx, bands)
        if ref_rej is not None:
            want = m
            break
    assert stop == want
    if stop < M:
        assert _judge_product(c, c.products[stop], f.measure(stop), ctx, bands) == ref_rej
        assert repr(ctx.stats.products[-1]) == repr(ref_ctx.stats.products[-1])  # NaN κ


# ---- freeze(): a calibration run's recorded numbers judged in slot order --------------------

def _calibrated(stats):
    """A calibration-mode Verifier over the MLP with one calibrated step whose recorded
    numbers are ``stats`` (as verify_step leaves them while judge=False)."""
    from verification.computation.instances.mlp import MLPComputation
    from verification.verifier.driver import Verifier
    c = MLPComputation((4, 8, 4), n_s=2, eta=1e-4)
    v = Verifier(c, h_D=bytes(32), n_records=2, k=1, n_steps=1, bands=None, seed=0,
                 w0_hashes=[bytes(32)] * c.n_w, calibrate=True)
    v.calibrated_steps.append(1)
    v.stats[1] = stats
    v.timings[1] = {}
    return v


# the MLP's two weights, standing for a linear weight (6a) and a glue weight (6b)
W_LIN, W_GLUE = "layers.0.weight", "layers.1.weight"


def _stats(rho_6a=1.0, rho_6b=1.0, kappa=1.0, res=0.5):
    from verification.verifier.context import ProductStat, StepStats, TensorStat
    s = StepStats()
    s.tensors.append(TensorStat(W_LIN, "6a", rho_6a))
    s.products.append(ProductStat(m=1, name="Y_1", cls="forward:Y_1", kappa=kappa,
                                  normalized=(res,)))
    s.tensors.append(TensorStat(W_GLUE, "6b", rho_6b))
    return s


def test_freeze_judges_a_glue_update_over_its_band():
    v = _calibrated(_stats(rho_6b=9.0))
    rej = v.freeze(Bands(tau=8.0, kappa_max=1e4, tau_w=4.0, source="file"))
    assert rej == Rejection(1, "6b", f"{W_GLUE}: ρ_max = 9 > τ_W = 4")
    assert v.rejection == rej


def test_freeze_order_is_6a_then_5_then_6b():
    bands = Bands(tau=8.0, kappa_max=1e4, tau_w=4.0, source="file")
    every = _stats(rho_6a=5.0, rho_6b=9.0, res=9.5)
    assert _calibrated(every).freeze(bands).check_id == "6a"
    no_6a = _stats(rho_6b=9.0, res=9.5)
    rej = _calibrated(no_6a).freeze(bands)
    assert rej.check_id == "5" and "challenge j=1" in rej.detail
    assert _calibrated(_stats()).freeze(bands) is None
    # a NaN ρ_max is not ≤ τ_W, so it rejects as the live check would
    assert _calibrated(_stats(rho_6b=math.nan)).freeze(bands).check_id == "6b"
    # a per-tensor τ_W judges that weight alone
    wide = Bands(tau=8.0, kappa_max=1e4, tau_w=4.0, tau_w_tensors={W_GLUE: 16.0},
                 source="file")
    assert _calibrated(_stats(rho_6b=9.0)).freeze(wide) is None
