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


def _verify(c, leaves, claimed, k=2):
    from verification.transcript.store import InMemoryStore
    from verification.verifier.driver import Verifier
    v = Verifier(c, k=k)
    rej = v.verify_step(1, InMemoryStore(leaves, claimed_root=claimed))
    return v, rej


def test_honest_step_accepts_with_stats(lib):
    c, step = _step(11)
    claimed = _root(c, step.leaves)
    v, rej = _verify(c, step.leaves, claimed)
    assert rej is None
    stats = v.stats[1].products
    assert [s.m for s in stats] == [s.m for s in c.products]
    assert all(max(s.normalized) <= 8.0 for s in stats)
    assert set(v.timings[1]) == {"2", "6a", "5", "2.root"}


def test_forged_product_rejects_at_check_5(lib):
    c, step = _step(12)
    spec = c.products[len(c.products) // 3]
    step.product(spec.m)[1, 2] += 8.0
    v, rej = _verify(c, step.leaves, _root(c, step.leaves))
    assert rej is not None and (rej.step, rej.check_id, rej.kind) == (1, "5", "failed")
    assert re.fullmatch(rf"P_{spec.m} \({re.escape(spec.name)}\), challenge j=1: normalized "
                        rf"residual \S+ > τ = 8", rej.detail), rej.detail
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
    i = c.w_t_index(name)
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
    from verification.transcript.store import InMemoryStore
    from verification.verifier.driver import Verifier
    c, step = _step(17)
    store = InMemoryStore(step.leaves, claimed_root=_root(c, step.leaves))
    step.leaves[c.n_s].add_(1.0)
    rej = Verifier(c, k=2).verify_step(1, store)
    assert rej is not None and (rej.check_id, rej.kind) == ("2", "malformed")
    assert "StoreMutationError" in rej.detail


def test_check_5_agrees_with_the_device_step_verifier(lib):
    from verification.verifier.step import DeviceStepVerifier
    c, step = _step(18, k=3)
    spec = c.products[5]
    step.product(spec.m)[0, 0] += 64.0  # well above a bf16 product's band
    claimed = _root(c, step.leaves)
    _, rej = _verify(c, step.leaves, claimed, k=3)
    out = DeviceStepVerifier(c, step.leaves, lambda s: step.operands[s.m], k=3).run(claimed)
    assert rej is not None and rej.check_id == "5" and out.check == "5"
    assert out.first_fail == spec.m - 1
    assert rej.detail.startswith(f"P_{spec.m} ({spec.name})")
