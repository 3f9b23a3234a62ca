"""Check 6a on the GPU: the update-identity kernel against the CPU oracle, and the check-level
function against the reference's wording.

The kernel's three outputs per weight — ``ρ_max`` (its float64 bits, NaN included), the first
non-finite entry and the first entry over ``τ_W`` — must equal the oracle's restatement of
``checks._update_identity_reference`` (checks.py:380-451) bit for bit, on the cases the
reference's own tests exercise (tests/verification/verifier/test_update_identity.py): honest
and exactly rounded steps, forged and tied entries, ``ρ`` at ``τ_W``, non-finite gradients and
updates, a scale that overflows, zero scales, an fp32 quotient that underflows, and
multi-part bf16 gradients.
"""

from __future__ import annotations

import math
import struct

import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
EPS_W, TAU_W, ETA = 2.0**-24, 4.0, 1e-3


def _bits(x: float) -> bytes | str:
    return "nan" if math.isnan(x) else struct.pack("<d", x)


def _honest(shape, seed=0, eta=ETA):
    gen = torch.Generator().manual_seed(seed)
    w = torch.randn(shape, generator=gen)
    g = torch.randn(shape, generator=gen)
    return w, torch.add(w, g, alpha=-eta), g


def _ulps(x, i, q):
    x = x.clone()
    for _ in range(q):
        x.view(-1)[i] = torch.nextafter(x.view(-1)[i], torch.tensor(math.inf, device=x.device))
    return x


def _run(lib, cases, eta=ETA, eps_w=EPS_W):
    """cases: [(w_t, w_next, parts, tau_w)] on the CPU; one plan over all of them."""
    from verification.commitment import native
    ws = [native.UpdateWeight(w.to(DEV).contiguous(), wn.to(DEV).contiguous(),
                              [p.to(DEV).contiguous() for p in parts], tau)
          for w, wn, parts, tau in cases]
    plan = lib.update_plan(ws, eta, eps_w)
    got = native.UpdatePlan.decode(plan.run())
    plan.close()
    for (w, wn, parts, tau), (rho, nf, ov) in zip(cases, got):
        want = O.update_identity(w, wn, parts, eta, eps_w, tau)
        assert _bits(rho) == _bits(want["rho_max"]), (rho, want["rho_max"])
        assert nf == want["first_nonfinite"] and ov == want["first_over"], (nf, ov, want)
    return got


def test_honest_and_exact_steps(lib):
    cases = []
    for seed, shape in enumerate([(48, 40), (7, 3, 33), (300,), (1,), (1000, 70)]):
        w, wn, g = _honest(shape, seed)
        cases.append((w, wn, [g], TAU_W))
        cases.append((w, w - ETA * g, [g], TAU_W))  # the reference's own rounding: ρ = 0
    got = _run(lib, cases)
    assert all(r[1] is None and r[2] is None for r in got)
    assert all(got[i][0] == 0.0 for i in range(1, len(cases), 2))


def test_forged_tied_and_threshold_entries(lib):
    w, _, g = _honest((40, 40), seed=3)
    tied = w - ETA * g
    for i in range(0, w.numel(), 7):
        tied = _ulps(tied, i, 1)
    w1, wn1, g1 = _honest((50, 30), seed=1)
    w2, wn2, g2 = _honest((20, 20), seed=2)
    forged2 = _ulps(wn2, 5, 5)
    rho = O.update_identity(w2, forged2, [g2], ETA, EPS_W, math.inf)["rho_max"]
    got = _run(lib, [(w, tied, [g], TAU_W), (w1, _ulps(wn1, 777, 9), [g1], TAU_W),
                     (w2, forged2, [g2], rho), (w2, forged2, [g2], math.nextafter(rho, 0.0))])
    assert 1.0 < got[0][0] <= 2.0
    assert got[1][2] == 777 and got[2][2] is None and got[3][2] == 5


@pytest.mark.parametrize("bad", [math.nan, math.inf, -math.inf])
def test_non_finite_gradient_and_update(lib, bad):
    w, wn, g = _honest((30, 30), seed=4)
    g = g.clone()
    g.view(-1)[123] = bad
    w5, wn5, g5 = _honest((30, 30), seed=5)
    wn5 = wn5.clone()
    wn5.view(-1)[17] = bad
    got = _run(lib, [(w, wn, [g], TAU_W), (w5, wn5, [g5], TAU_W)])
    assert got[0][1] == 123 and got[1][1] == 17


def test_overflow_zero_scale_and_underflow(lib):
    w, wn, g = _honest((10, 10), seed=6, eta=1.0)
    w, wn, g = w.clone(), wn.clone(), g.clone()
    w.view(-1)[9] = g.view(-1)[9] = 3e38
    wn.view(-1)[9] = 0.0
    got = _run(lib, [(w, wn, [g], TAU_W)], eta=1.0)
    assert got[0][1] == 9
    w, wn, g = _honest((16, 16), seed=7)
    w, wn, g = w.clone(), wn.clone(), g.clone()
    for i in (0, 40, 255):
        w.view(-1)[i] = g.view(-1)[i] = wn.view(-1)[i] = 0.0
    zero_ok = (w.clone(), wn.clone(), [g.clone()], TAU_W)
    wn.view(-1)[40] = 1e-30
    uw, ug, uwn = torch.zeros(4, 4), torch.zeros(4, 4), torch.zeros(4, 4)
    uw.view(-1)[9] = ug.view(-1)[9] = 1e38
    uwn.view(-1)[9] = 1.4e-45
    got = _run(lib, [zero_ok, (w, wn, [g], TAU_W)])
    assert got[0][2] is None and got[1][0] == math.inf and got[1][2] == 40
    got = _run(lib, [(uw, uwn, [ug], TAU_W)], eta=1.0)
    assert got[0][2] is None and 0.0 < got[0][0] < 1e-70


def test_multi_part_bf16_gradients_and_many_blocks(lib):
    gen = torch.Generator().manual_seed(11)
    shape = (1536, 1000)  # ~375 blocks of 4096 entries
    parts = [torch.randn(shape, generator=gen).to(torch.bfloat16) for _ in range(3)]
    w = torch.randn(shape, generator=gen)
    g = O.chain_gradient(parts)
    wn = torch.add(w, g, alpha=-ETA)
    forged = _ulps(wn, shape[0] * shape[1] - 3, 40)
    mixed = [parts[0], parts[1].float(), parts[2]]
    got = _run(lib, [(w, wn, parts, TAU_W), (w, forged, parts, TAU_W), (w, wn, mixed, TAU_W)])
    assert got[0][2] is None and got[1][2] == shape[0] * shape[1] - 3


def test_empty_weight(lib):
    w = torch.zeros(0, 5)
    got = _run(lib, [(w, w.clone(), [w.clone()], TAU_W), (*_honest((3,), 1)[:2],
                                                          [_honest((3,), 1)[2]], TAU_W)])
    assert got[0] == (0.0, None, None)


# ---- the check-level function ------------------------------------------------------------

def _step(seed):
    from verification.computation.instances.decoder import DecoderComputation
    from verification.prover.synthetic import synthetic_step
    c = DecoderComputation(L=2, d=64, d_f=128, n_h=4, n_kv=2, n_v=160, n_s=2, n=32,
                           qkv_bias=True, compute_dtype=torch.bfloat16)
    step = synthetic_step(c, seed=seed, operands=True)
    c.use_operands(step.replay())
    return c, step


def _root(c, leaves):
    want = []
    for i, obj in enumerate(leaves):
        if i < c.n_s:
            want.append(O.hash_leaf(O.encode_record(obj.ids, obj.targets, obj.mask)))
        else:
            tag = O.TAG_PRODUCT if c.n_s + c.n_w <= i < c.n_s + c.n_w + c.M else O.TAG_WEIGHT
            want.append(O.tensor_leaf_hash(tag, obj.cpu()))
    return O.merkle_root(want)


def _verify(c, leaves, calibrate=False):
    from conftest import started_verifier
    from verification.transcript.store import InMemoryStore
    v = started_verifier(c, leaves, k=2, calibrate=calibrate)
    return v, v.verify_step(1, InMemoryStore(leaves, claimed_root=_root(c, leaves)))


def _oracle_weight(c, leaves, name, tau=TAU_W):
    parts = [leaves[c.product_index(m)] for m in c.linear_weights[name]]
    return O.update_identity(leaves[c.w_t_index(name)], leaves[c.w_next_index(name)], parts,
                             c.eta, EPS_W, tau)


def test_check_6a_honest_step_records_every_weight(lib):
    c, step = _step(21)
    v, rej = _verify(c, step.leaves)
    assert rej is None
    tensors = v.stats[1].tensors
    assert [t.weight for t in tensors] == list(c.linear_weights)
    assert all(t.check_id == "6a" and t.rho_max <= TAU_W for t in tensors)
    for t in tensors[::5]:
        assert _bits(t.rho_max) == _bits(_oracle_weight(c, step.leaves, t.weight)["rho_max"])
    assert list(v.timings[1]) == (["read", "serve", "plans", "gpu", "judge"] if v.overlapped
                                  else ["7", "2", "6a", "5", "6b", "2.root"])


def test_check_6a_forged_update_rejects_with_the_reference_wording(lib):
    c, step = _step(22)
    names = list(c.linear_weights)
    name = names[len(names) // 2]
    leaves = list(step.leaves)
    i = c.w_next_index(name)
    leaves[i] = _ulps(leaves[i], 17, 64)
    v, rej = _verify(c, leaves)
    want = _oracle_weight(c, leaves, name)
    j = want["first_over"]
    r, s = float(want["r"][j]), float(want["scale"][j])
    assert rej is not None and (rej.step, rej.check_id, rej.kind) == (1, "6a", "failed")
    assert rej.detail == (f"{name}: entry {j} has |R| = {r:.3e}, bound {TAU_W * s:.3e} "
                          f"(ρ_max = {want['rho_max']:.3g}, τ_W = {TAU_W:g})")
    assert [t.weight for t in v.stats[1].tensors] == names[:names.index(name) + 1]
    assert v.stats[1].products == []  # check 5 did not run
    # calibration records and never judges the band ...
    v, rej = _verify(c, leaves, calibrate=True)
    assert rej is None and len(v.stats[1].tensors) == len(names)


def test_check_6a_non_finite_update_rejects_in_both_modes(lib):
    """Finite leaves (a non-finite leaf is malformed at check 2 already) whose residual
    overflows: W_t = 3e38 and W_{t+1} = −3e38 make W_{t+1} − (W_t − η·G) = −inf."""
    c, step = _step(23)
    name = list(c.linear_weights)[3]
    leaves = list(step.leaves)
    for idx, v in ((c.w_t_index(name), 3e38), (c.w_next_index(name), -3e38)):
        leaves[idx] = leaves[idx].clone()
        leaves[idx].view(-1)[5] = v
    want = _oracle_weight(c, leaves, name)
    r, s = float(want["r"][5]), float(want["scale"][5])
    for calibrate in (False, True):
        _, rej = _verify(c, leaves, calibrate=calibrate)
        assert rej is not None and rej.check_id == "6a"
        assert rej.detail == (f"{name}: entry 5 has a non-finite residual or bound "
                              f"(|R| = {r:.3e}, scale {s:.3e})")
