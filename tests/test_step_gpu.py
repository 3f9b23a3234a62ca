"""The whole device-resident step (check 2 hashing + root, check 5 rows + verdicts) on two
streams, against the CPU oracle, and the stage entry points against the one-call runs.

Tolerances: digests, roots, first-bad/first-fail indices and verdict codes bit for bit; the
Freivalds rows of the step as in the Freivalds tests (non-negative sums relative 1e-5,
residuals of bf16 products relative 1e-4 with an absolute floor of 2 band units).
"""

from __future__ import annotations


import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu
BF16, FP32 = 2.0**-8, 2.0**-24


def _tiny(seed=1, qkv_bias=True):
    from verification.computation.instances.decoder import DecoderComputation
    from verification.prover.synthetic import synthetic_step
    c = DecoderComputation(L=2, d=64, d_f=128, n_h=4, n_kv=2, n_v=160, n_s=2, n=32,
                           qkv_bias=qkv_bias, compute_dtype=torch.bfloat16)
    return c, synthetic_step(c, seed=seed, operands=True)


def _oracle_root(c, leaves):
    want = []
    for i, obj in enumerate(leaves):
        if i < c.n_s:
            want.append(O.hash_leaf(O.encode_record(obj.ids, obj.targets, obj.mask)))
        else:
            tag = O.TAG_PRODUCT if c.n_s + c.n_w <= i < c.n_s + c.n_w + c.M else O.TAG_WEIGHT
            want.append(O.tensor_leaf_hash(tag, obj.cpu()))
    return O.merkle_root(want)


def _verifier(c, step, k=2):
    from verification.verifier.step import DeviceStepVerifier
    return DeviceStepVerifier(c, step.leaves, lambda s: step.operands[s.m], k=k)


def test_honest_step_accepts_and_matches_oracle(lib):
    c, step = _tiny()
    v = _verifier(c, step)
    claimed = _oracle_root(c, step.leaves)
    out = v.run(claimed)
    assert out.root == claimed
    assert out.first_bad == c.n_leaves and out.first_fail == c.M
    assert out.check is None, out.detail
    codes = out.codes.cpu()
    assert (codes[:, 0] == 0).all()
    # the rows equal the oracle's measurement of every product under the claimed root
    rows = out.rows.cpu().tolist()
    for i, spec in enumerate(c.products):
        a, b = step.operands[spec.m]
        p = step.product(spec.m)
        bias = None
        if spec.bias is not None:
            bias = step.w_t(spec.bias).to(torch.bfloat16).float().cpu()
        r = O.challenge_matrices(claimed, [spec.m], 2, p.shape[1])[0]
        af, bf, pf = a.float().cpu(), b.float().cpu(), p.float().cpu()
        want = O.measure_product_row(af, bf, pf, r, bias)
        for col in range(5):
            assert rows[i][col] == pytest.approx(want[col], rel=1e-5, abs=1e-30), (i, col)
        ref64 = O.measure_row_f64(af, bf, pf, r, bias)
        mp = O.finish_row(ref64, q=spec.q, n=af.shape[0], eps_in=BF16, eps_acc=FP32,
                          biased=bias is not None)
        for j in range(2):
            assert rows[i][5 + j] == pytest.approx(ref64[5 + j], rel=1e-4, abs=2 * mp["unit"])


def test_planted_product_error_rejects_at_that_product(lib):
    c, step = _tiny(seed=2)
    v = _verifier(c, step)
    bad_m = c.products[len(c.products) // 2].m
    p = step.product(bad_m)
    p[3, 5] += 4.0  # a wrong entry the prover commits to
    claimed = _oracle_root(c, step.leaves)  # the cheating prover's own root
    out = v.run(claimed)
    assert out.root == claimed
    assert out.check == "5", out.detail
    assert out.first_fail == next(i for i, s in enumerate(c.products) if s.m == bad_m)
    assert int(out.codes[out.first_fail, 0]) == 3


def test_nonfinite_leaf_is_check_2(lib):
    c, step = _tiny(seed=3)
    v = _verifier(c, step)
    w_idx = c.n_s + 1
    step.leaves[w_idx].view(-1)[7] = float("inf")
    out = v.run(bytes(32))
    assert out.check == "2" and out.first_bad == w_idx, out.detail


def test_wrong_claimed_root_is_check_2_at_the_end(lib):
    c, step = _tiny(seed=4)
    v = _verifier(c, step)
    honest = _oracle_root(c, step.leaves)
    out = v.run(bytes(b ^ 1 for b in honest))
    assert out.root == honest
    assert out.first_fail == c.M  # honest products pass under any key
    assert out.check == "2", out.detail


def test_stage_entry_points_equal_one_call_runs(lib):
    from verification.commitment import native
    c, step = _tiny(seed=5)
    v = _verifier(c, step, k=3)
    claimed = _oracle_root(c, step.leaves)
    d1, _ = v.hasher.digests()
    key = torch.frombuffer(bytearray(claimed), dtype=torch.uint8).cuda()
    r1 = v.plan.rows(key)
    d2 = torch.empty_like(d1)
    bad = torch.empty(1, dtype=torch.int32, device="cuda")
    for st in range(len(native.LeafPlan.STAGES)):
        v.hasher.plan.run_stage(st, d2, bad)
    r2 = torch.empty_like(r1)
    for st in range(len(native.FvPlan.STAGES)):
        v.plan.run_stage(st, key, r2)
    torch.cuda.synchronize()
    assert torch.equal(d1, d2)
    assert int(bad.item()) == c.n_leaves
    assert torch.equal(r1.view(torch.int64), r2.view(torch.int64))
    with pytest.raises(ValueError):  # past stage 3's two parts (8, 9)
        v.plan.run_stage(native.FvPlan.TWINS + 1, key, r2)
    with pytest.raises(ValueError):
        v.hasher.plan.run_stage(-1, d2, bad)
