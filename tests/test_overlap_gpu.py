"""The overlapped path of ``Verifier.verify_step`` against the slots run one at a time
(reference verification/verifier/driver.py:223-263, checks.py:204-272, 576-658).

An honest step must be accepted on the overlapped path with the kept hashes the slots give
and their statistics (check 5's to fp32 rounding of the fused P-pass sums); a second verifier on the same layout must reuse its plans. Every cheat
must reject with the same ``Rejection`` as the serial slots (the overlapped path leaves every
rejection to them): a non-finite leaf (check 2, malformed), a forged product the prover
re-roots (check 5), a claimed root that is not the leaves' (check 2 last), an operand the
replay cannot serve (check 5, malformed), a W_t that is not the agreed W_0 (check 0) and a
forged W_{t+1} (check 6a). The step's dimensions let the twin pass take the attention
probabilities and δS (n = 128), and the chunk kernel the P-pass sums of the rows of 1 KiB.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _step(seed):
    from verification.computation.instances.decoder import DecoderComputation
    from verification.prover.synthetic import synthetic_step
    c = DecoderComputation(L=2, d=128, d_f=512, n_h=2, n_kv=1, n_v=512, n_s=2, n=128,
                           qkv_bias=True, compute_dtype=torch.bfloat16)
    step = synthetic_step(c, seed=seed, operands=True)
    return c, step


def _root(c, leaves):
    from verification.commitment.leaves import commit_leaves_device
    return commit_leaves_device(c, leaves).root


def _run(c, leaves, claimed, *, overlap, w0=None, replay=None, plans=None):
    from conftest import started_verifier
    from verification.transcript.store import InMemoryStore
    c.use_operands(replay)
    v = started_verifier(c, w0 if w0 is not None else leaves, k=2, overlap=overlap)
    if plans is not None:
        v.plans = plans
    rej = v.verify_step(1, InMemoryStore(leaves, claimed_root=claimed))
    return v, rej


def _stats(v):
    s = v.stats[1]
    return ([(p.m, p.kappa, p.normalized, p.p_norm, p.nu, p.p_abs1, p.u) for p in s.products],
            [(t.weight, t.check_id, t.rho_max) for t in s.tensors])


def _close(fast, slow):
    """The overlapped path's statistics against the slots': the same products and weights;
    check 6's ρ_max bit for bit; check 5's numbers to fp32 rounding, since the fused chunk
    kernel takes the P-pass sums in another order (the sums to 1e-6 relative, as the fused
    plan's tests hold them, the normalized residuals to 1e-3 of a band unit)."""
    (pf, tf), (ps, ts) = _stats(fast), _stats(slow)
    assert tf == ts
    assert [p[0] for p in pf] == [p[0] for p in ps]
    for a, b in zip(pf, ps):
        assert a[1] == pytest.approx(b[1], rel=1e-5), a[0]
        assert a[2] == pytest.approx(b[2], rel=1e-3, abs=1e-3), a[0]
        assert a[3:] == pytest.approx(b[3:], rel=1e-6), a[0]


def test_honest_step_is_accepted_on_the_overlapped_path(lib):
    c, step = _step(1)
    claimed = _root(c, step.leaves)
    fast, rej = _run(c, step.leaves, claimed, overlap=True, replay=step.replay())
    assert rej is None and fast.overlapped == [1] and fast.serial == []
    entry = fast.plans.overlap.entry
    assert entry.fv.twins > 0 and entry.leaf.fused > 0
    slow, rej = _run(c, step.leaves, claimed, overlap=False, replay=step.replay())
    assert rej is None and slow.serial == [1]
    _close(fast, slow)
    assert fast._chain == slow._chain
    # a second verifier on the same transcript reuses the plans
    again, rej = _run(c, step.leaves, claimed, overlap=True, replay=step.replay(),
                      plans=fast.plans)
    assert rej is None and again.overlapped == [1]
    assert again.plans.overlap.hits == 1 and again.plans.overlap.builds == 1
    assert _stats(again) == _stats(fast)
    fast.close()
    slow.close()


def _same(c, leaves, claimed, **kw):
    fast, got = _run(c, leaves, claimed, overlap=True, **kw)
    slow, want = _run(c, leaves, claimed, overlap=False, **kw)
    assert got is not None and got == want, (got, want)
    assert fast.serial == [1] and fast.overlapped == []
    assert _stats(fast) == _stats(slow)  # both from the slots
    fast.close()
    slow.close()
    return got


def test_a_non_finite_leaf_rejects_as_the_slots_do(lib):
    c, step = _step(2)
    claimed = _root(c, step.leaves)
    leaves = list(step.leaves)
    i = c.product_index(c.products[len(c.products) // 2].m)
    leaves[i] = leaves[i].clone()
    leaves[i].view(-1)[5] = float("nan")
    rej = _same(c, leaves, claimed, replay=step.replay())
    assert rej.check_id == "2" and rej.kind == "malformed"


def test_a_forged_product_rejects_as_the_slots_do(lib):
    c, step = _step(3)
    leaves = list(step.leaves)
    spec = next(s for s in c.products if s.name.startswith("L1.dV"))
    i = c.product_index(spec.m)
    leaves[i] = leaves[i].clone()
    leaves[i][7, 3] += 64.0
    rej = _same(c, leaves, _root(c, leaves), replay=step.replay())
    assert rej.check_id == "5" and f"P_{spec.m} " in rej.detail


def test_a_wrong_root_rejects_as_the_slots_do(lib):
    c, step = _step(4)
    claimed = bytes(b ^ 0x5A for b in _root(c, step.leaves))
    rej = _same(c, step.leaves, claimed, replay=step.replay())
    assert rej.check_id == "2" and "recomputed root" in rej.detail


def test_a_serving_error_rejects_as_the_slots_do(lib):
    from verification.prover.synthetic import CapturedReplay
    from verification.transcript.errors import TranscriptFormatError
    c, step = _step(5)
    bad_m = next(s for s in c.products if s.name.startswith("L2.dQ")).m

    class Failing(CapturedReplay):
        def operands(self, m):
            if m == bad_m:
                raise TranscriptFormatError(f"operand file of product {m} is truncated")
            return super().operands(m)

    claimed = _root(c, step.leaves)
    rej = _same(c, step.leaves, claimed, replay=Failing(step.operands, step.groups))
    assert rej.check_id == "5" and rej.kind == "malformed" and "truncated" in rej.detail


def test_chain_and_update_failures_reject_as_the_slots_do(lib):
    c, step = _step(6)
    claimed = _root(c, step.leaves)
    w0 = list(step.leaves)
    name = c.weight_names[3]
    w0[c.w_t_index(name)] = w0[c.w_t_index(name)] + 1.0
    rej = _same(c, step.leaves, claimed, replay=step.replay(), w0=w0)
    assert rej.check_id == "0" and name in rej.detail
    leaves = list(step.leaves)
    lin = next(iter(c.linear_weights))
    j = c.w_next_index(lin)
    leaves[j] = leaves[j].clone()
    leaves[j].view(-1)[11] += 0.5
    rej = _same(c, leaves, _root(c, leaves), replay=step.replay())
    assert rej.check_id == "6a" and lin in rej.detail


def test_plans_run_again_only_on_the_same_layout(lib):
    """The overlapped path keeps its last step's plans: the same tensors run them again; a
    product forged in place (same layout) is left to the slots, which reject it at check 5;
    a product moved to another buffer builds them again; new records at the same addresses
    keep them (records are staged every step)."""
    from conftest import started_verifier
    from setup.records import Record
    from verification.transcript.store import InMemoryStore
    c, step = _step(7)
    c.use_operands(step.replay())
    claimed = _root(c, step.leaves)

    def run(leaves, root, plans=None):
        v = started_verifier(c, leaves, k=2)
        if plans is not None:
            v.plans = plans
        return v, v.verify_step(1, InMemoryStore(leaves, claimed_root=root))

    v1, rej = run(step.leaves, claimed)
    ov = v1.plans.overlap
    assert rej is None and v1.overlapped == [1] and (ov.builds, ov.hits) == (1, 0)
    v2, rej = run(step.leaves, claimed, v1.plans)
    assert rej is None and v2.overlapped == [1] and (ov.builds, ov.hits) == (1, 1)
    spec = c.products[9]
    honest = step.product(spec.m)[0, 1].clone()
    step.product(spec.m)[0, 1] += 64.0
    v3, rej = run(step.leaves, _root(c, step.leaves), v1.plans)
    assert rej is not None and rej.check_id == "5" and rej.detail.startswith(f"P_{spec.m} (")
    assert v3.serial == [1] and (ov.builds, ov.hits) == (1, 2)
    step.product(spec.m)[0, 1] = honest
    i = c.product_index(spec.m)
    step.leaves[i] = step.leaves[i].clone()
    v4, rej = run(step.leaves, claimed, v1.plans)
    assert rej is None and v4.overlapped == [1] and (ov.builds, ov.hits) == (2, 2)
    r = step.leaves[0]
    step.leaves[0] = Record(torch.flip(r.ids, [0]).contiguous(), r.targets, r.mask)
    v5, rej = run(step.leaves, _root(c, step.leaves), v1.plans)
    assert rej is None and v5.overlapped == [1] and (ov.builds, ov.hits) == (2, 3)
    v5.close()


def test_moved_operands_over_the_same_leaves(lib):
    """A replay rebuilt for the next step serves its operands from new buffers while the
    leaves stay where they were: the kept leaf plan still hashes every leaf, the step is
    measured on a Freivalds plan of its own and accepted on the overlapped path with the same
    kept hashes; the kept plans stay for the next step."""
    from verification.prover.synthetic import CapturedReplay
    c, step = _step(8)
    claimed = _root(c, step.leaves)
    v1, rej = _run(c, step.leaves, claimed, overlap=True, replay=step.replay())
    assert rej is None and v1.overlapped == [1]
    moved = {m: (a.clone(), b.clone()) for m, (a, b) in step.operands.items()}
    v2, rej = _run(c, step.leaves, claimed, overlap=True, replay=CapturedReplay(moved),
                   plans=v1.plans)
    assert rej is None and v2.overlapped == [1], v2.plans.overlap.declined
    assert v2._chain == v1._chain
    assert v2.plans.overlap.builds == 1 and v2.plans.overlap.hits == 0
    slow, rej = _run(c, step.leaves, claimed, overlap=False, replay=CapturedReplay(moved))
    assert rej is None
    _close(v2, slow)
    v3, rej = _run(c, step.leaves, claimed, overlap=True, replay=step.replay(),
                   plans=v1.plans)
    assert rej is None and v3.overlapped == [1]
    assert (v3.plans.overlap.builds, v3.plans.overlap.hits) == (1, 1)
    for v in (v1, v2, v3, slow):
        v.close()
