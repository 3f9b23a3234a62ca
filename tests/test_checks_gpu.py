"""Checks 2, 5 and 2.root through the reference's check-level API, on a transcript in HBM.

Expected outcomes follow the reference's cheat matrix for these checks
(tests/verification/verifier/test_verifier.py): an honest step accepts; a wrong product entry
the prover commits to rejects at check 5 ("failed", at that product); NaN/Inf or a leaf of the
wrong shape rejects at check 2 ("malformed"); a claimed root that is not the leaves' root
rejects at check 2 last; a claimed root that is not a digest is malformed at check 2. The
root is checked against the CPU oracle bit for bit, and check 5's first failure against the
device verdict kernel (check_5_matmuls raises if the two disagree).
"""

from __future__ import annotations

import re

import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu


def _step(seed, k=2):
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


def _verify(c, leaves, claimed, k=2, w0_leaves=None, **kw):
    from conftest import started_verifier
    from verification.transcript.store import InMemoryStore
    v = started_verifier(c, w0_leaves if w0_leaves is not None else leaves, k=k, **kw)
    rej = v.verify_step(1, InMemoryStore(leaves, claimed_root=claimed))
    return v, rej


@pytest.mark.parametrize("overlap", [True, False])
def test_honest_step_accepts_with_stats(lib, overlap):
    c, step = _step(11)
    claimed = _root(c, step.leaves)
    v, rej = _verify(c, step.leaves, claimed, overlap=overlap)
    assert rej is None
    stats = v.stats[1].products
    assert [s.m for s in stats] == [s.m for s in c.products]
    assert all(max(s.normalized) <= 8.0 for s in stats)
    if overlap:  # accepted on the overlapped path, timed by phase
        assert v.overlapped == [1]
        assert set(v.timings[1]) == {"read", "serve", "plans", "gpu", "judge"}
    else:
        assert v.serial == [1]
        assert set(v.timings[1]) == {"7", "2", "6a", "5", "6b", "2.root"}
    assert v.stats[1].operands_from_prover


def test_forged_product_rejects_at_check_5(lib):
    c, step = _step(12)
    spec = c.products[len(c.products) // 3]
    step.product(spec.m)[1, 2] += 64.0
    v, rej = _verify(c, step.leaves, _root(c, step.leaves))
    assert rej is not None and (rej.step, rej.check_id, rej.kind) == (1, "5", "failed")
    assert re.fullmatch(rf"P_{spec.m} \({re.escape(spec.name)}\), challenge j=[12]: "
                        rf"normalized residual \S+ > τ = 8", rej.detail), rej.detail
    assert v.stats[1].products[-1].m == spec.m  # judged up to the failing product


def test_non_finite_leaf_is_malformed_at_check_2(lib):
    c, step = _step(13)
    i = c.product_index(c.products[-1].m)
    step.leaves[i].view(-1)[0] = float("nan")
    _, rej = _verify(c, step.leaves, bytes(32))
    assert rej is not None and (rej.check_id, rej.kind) == ("2", "malformed")
    assert rej.detail == "malformed prover data: NonFiniteError: float tensor contains NaN or Inf"


def test_wrong_shape_leaf_is_malformed_at_check_2(lib):
    c, step = _step(14)
    leaves = list(step.leaves)
    name = next(n for n in c.weight_names if len(c.weight_shapes[n]) == 2)
    i = c.w_next_index(name)
    leaves[i] = leaves[i].reshape(-1)
    _, rej = _verify(c, leaves, bytes(32))
    assert rej is not None and (rej.check_id, rej.kind) == ("2", "malformed")
    assert rej.detail.startswith("malformed prover data: LeafShapeError: leaf ")


def test_wrong_root_rejects_at_check_2_last(lib):
    c, step = _step(15)
    honest = _root(c, step.leaves)
    claimed = bytes([honest[0] ^ 0x80]) + honest[1:]
    v, rej = _verify(c, step.leaves, claimed)
    assert rej is not None and (rej.check_id, rej.kind) == ("2", "failed")
    assert rej.detail == f"recomputed root {honest.hex()[:16]}… != claimed {claimed.hex()[:16]}…"
    assert len(v.stats[1].products) == c.M  # check 5 ran first, on the claimed root


def test_claimed_root_not_a_digest_is_malformed(lib):
    c, step = _step(16)
    _, rej = _verify(c, step.leaves, b"\x00" * 31)
    assert rej is not None and (rej.check_id, rej.kind, rej.detail) == \
        ("2", "malformed", "claimed root is not a 32-byte digest")


def test_mutation_after_handoff_is_malformed(lib):
    from conftest import started_verifier
    from verification.transcript.store import InMemoryStore
    c, step = _step(17)
    v = started_verifier(c, step.leaves, k=2)
    store = InMemoryStore(step.leaves, claimed_root=_root(c, step.leaves))
    step.leaves[c.product_index(1)].add_(1.0)
    rej = v.verify_step(1, store)
    assert rej is not None and (rej.check_id, rej.kind) == ("2", "malformed")
    assert "StoreMutationError" in rej.detail
    # a W_t leaf is read first by check 0 on the first step
    c, step = _step(17)
    v = started_verifier(c, step.leaves, k=2)
    store = InMemoryStore(step.leaves, claimed_root=_root(c, step.leaves))
    step.leaves[c.n_s].add_(1.0)
    rej = v.verify_step(1, store)
    assert rej is not None and (rej.check_id, rej.kind) == ("0", "malformed")
    assert "StoreMutationError" in rej.detail


def test_w_t_other_than_w0_rejects_at_check_0(lib):
    c, step = _step(19)
    w0 = list(step.leaves)
    name = c.weight_names[3]
    w0[c.w_t_index(name)] = w0[c.w_t_index(name)] + 1.0
    _, rej = _verify(c, step.leaves, _root(c, step.leaves), w0_leaves=w0)
    assert rej is not None and (rej.step, rej.check_id, rej.kind) == (1, "0", "failed")
    assert rej.detail == f"W_t[{name}] differs from the agreed W_0"


def test_two_steps_chain_and_end_run(lib):
    """Step 2 starts from step 1's W_{t+1} (check 7); check 8 compares the last W_{t+1} with
    the agreed final weights and counts the steps."""
    from conftest import started_verifier
    from verification.computation.interface import chain_gradient
    from verification.transcript.store import InMemoryStore
    c, step = _step(20)
    nxt = list(step.leaves)
    for name in c.weight_names:  # same products; W_t moves on, W_{t+1} follows check 6a
        w_t = step.leaves[c.w_next_index(name)]
        nxt[c.w_t_index(name)] = w_t
        if name in c.linear_weights:
            g = chain_gradient((step.leaves[c.product_index(m)]
                                for m in c.linear_weights[name]), torch.float32)
            nxt[c.w_next_index(name)] = torch.add(w_t, g, alpha=-c.eta)
        else:
            nxt[c.w_next_index(name)] = w_t - 1e-4
    final = {n: nxt[c.w_next_index(n)].clone() for n in c.weight_names}
    v = started_verifier(c, step.leaves, k=2, n_steps=2)
    for t, leaves in ((1, step.leaves), (2, nxt)):
        assert v.verify_step(t, InMemoryStore(leaves, claimed_root=_root(c, leaves))) is None
    verdict = v.end_run(final)
    assert verdict.accepted and verdict.steps_verified == 2 and verdict.rejection is None
    # a second step that does not start from step 1's W_{t+1} fails check 7
    v = started_verifier(c, step.leaves, k=2, n_steps=2)
    assert v.verify_step(1, InMemoryStore(step.leaves, claimed_root=_root(c, step.leaves))) \
        is None
    rej = v.verify_step(2, InMemoryStore(step.leaves, claimed_root=_root(c, step.leaves)))
    assert rej is not None and (rej.step, rej.check_id, rej.kind) == (2, "7", "failed")
    assert rej.detail == f"W_t[{c.weight_names[0]}] differs from W_{{t+1}} of step 1"
    # a run that stops early, or ends on other weights, fails check 8
    v = started_verifier(c, step.leaves, k=2, n_steps=2)
    assert v.verify_step(1, InMemoryStore(step.leaves, claimed_root=_root(c, step.leaves))) \
        is None
    verdict = v.end_run(final)
    assert not verdict.accepted and verdict.rejection.check_id == "8"
    assert verdict.rejection.detail == "1 steps verified, the run declares T = 2"
    v = started_verifier(c, step.leaves, k=2, n_steps=1)
    assert v.verify_step(1, InMemoryStore(step.leaves, claimed_root=_root(c, step.leaves))) \
        is None
    verdict = v.end_run(final)
    assert verdict.rejection.detail == \
        f"final W_T[{c.weight_names[0]}] differs from the agreed weights"


def test_serving_error_after_a_forged_product(lib):
    """A serving error at product m is raised only after the products before m are judged
    (reference checks.py:613-650): with a forged product k < m the step rejects at k as
    "failed" and keeps the error for the record; without it the error is check 5's malformed
    rejection."""
    from verification.transcript.errors import TranscriptFormatError
    from verification.transcript.store import InMemoryStore

    class Failing:
        prover_supplied = True

        def __init__(self, inner, m):
            self.inner, self.m = inner, m

        def operands(self, m):
            if m == self.m:
                raise TranscriptFormatError(f"operands of product {m} unreadable")
            return self.inner.operands(m)

    for forged in (True, False):
        c, step = _step(21)
        k_spec, m_spec = c.products[10], c.products[40]
        if forged:
            step.product(k_spec.m)[1, 2] += 8.0
        c.use_operands(Failing(step.replay(), m_spec.m))
        from conftest import started_verifier
        v = started_verifier(c, step.leaves, k=2, trust_prover_operands=True)
        store = InMemoryStore(step.leaves, claimed_root=_root(c, step.leaves))
        rej = v.verify_step(1, store)
        assert rej is not None and rej.check_id == "5"
        if forged:
            assert rej.kind == "failed" and rej.detail.startswith(f"P_{k_spec.m} ")
            assert [s.m for s in v.stats[1].products][-1] == k_spec.m
        else:
            assert rej.kind == "malformed"
            assert rej.detail == (f"malformed prover data: TranscriptFormatError: operands of "
                                  f"product {m_spec.m} unreadable")
            assert [s.m for s in v.stats[1].products] == [s.m for s in c.products[:40]]


def test_plans_kept_between_steps_run_again_only_on_the_same_layout(lib):
    """The slots run one at a time (``overlap=False``; the overlapped path's own plans are
    tested in test_overlap_gpu.py) keep the last step's leaf and Freivalds plans. A step with
    the same layout
    (here the same tensors) runs them again with the same hashes and statistics; a product
    changed in place, at the same address, still rejects at check 5; a product moved to
    another buffer makes check 2's leaf plan and the Freivalds plan be built again."""
    from conftest import started_verifier
    from verification.transcript.store import InMemoryStore
    c, step = _step(21)
    claimed = _root(c, step.leaves)
    v1 = started_verifier(c, step.leaves, k=2, overlap=False)
    assert v1.verify_step(1, InMemoryStore(step.leaves, claimed_root=claimed)) is None
    cache = v1.plans
    assert (cache.builds, cache.hits) == (3, 0)  # check 7's and 2's leaf plans, Freivalds
    v2 = started_verifier(c, step.leaves, k=2, overlap=False)
    v2.plans = cache
    assert v2.verify_step(1, InMemoryStore(step.leaves, claimed_root=claimed)) is None
    assert (cache.builds, cache.hits) == (3, 3)
    assert [repr(s) for s in v2.stats[1].products] == [repr(s) for s in v1.stats[1].products]

    spec = c.products[7]
    honest = step.product(spec.m)[0, 1].clone()
    step.product(spec.m)[0, 1] += 8.0  # forged in place: the layout is unchanged
    v3 = started_verifier(c, step.leaves, k=2, overlap=False)
    v3.plans = cache
    rej = v3.verify_step(1, InMemoryStore(step.leaves, claimed_root=_root(c, step.leaves)))
    assert rej is not None and (rej.check_id, rej.kind) == ("5", "failed"), rej
    assert rej.detail.startswith(f"P_{spec.m} ("), rej.detail
    assert (cache.builds, cache.hits) == (3, 6)

    step.product(spec.m)[0, 1] = honest
    i = c.product_index(spec.m)
    step.leaves[i] = step.leaves[i].clone()  # the same bytes in another buffer
    v4 = started_verifier(c, step.leaves, k=2, overlap=False)
    v4.plans = cache
    assert v4.verify_step(1, InMemoryStore(step.leaves, claimed_root=claimed)) is None
    assert (cache.builds, cache.hits) == (5, 7)
    assert [repr(s) for s in v4.stats[1].products] == [repr(s) for s in v1.stats[1].products]
    v4.close()


def test_new_records_keep_check_2s_plan(lib):
    """Records are hashed as their own batch, so a step with other records over the same
    tensor buffers still reuses check 2's leaf plan (the slots one at a time); the new root is
    the oracle's."""
    from conftest import started_verifier
    from setup.records import Record
    from verification.transcript.store import InMemoryStore
    c, step = _step(22)
    v1 = started_verifier(c, step.leaves, k=2, overlap=False)
    assert v1.verify_step(1, InMemoryStore(step.leaves, claimed_root=_root(c, step.leaves))) \
        is None
    cache = v1.plans
    r = step.leaves[0]
    step.leaves[0] = Record(torch.flip(r.ids, [0]).contiguous(), r.targets, r.mask)
    claimed = _root(c, step.leaves)
    v2 = started_verifier(c, step.leaves, k=2, overlap=False)
    v2.plans = cache
    assert v2.verify_step(1, InMemoryStore(step.leaves, claimed_root=claimed)) is None
    assert (cache.builds, cache.hits) == (3, 3)
    assert v2.stats[1].products  # check 5 ran on the cached Freivalds plan
