"""The prover on the GPU, and its steps verified from the committed leaves alone (reference
tests/verification/test_m1_smoke.py: an honest MLP step accepts, a perturbed product rejects;
the decoder's replay, reference decoder.py:1142-1751).

The products stay in HBM (the capture keeps each op's own output) and the commit hashes every
leaf there; the root must equal the CPU oracle's over the same leaves. The verifier then
rebuilds every operand from the committed leaves (``MLPReplay``, no captured operands) and
must accept the honest step through ``Verifier`` and ``DeviceStepVerifier`` alike, and reject
a step whose committed product was changed at check 5, and one whose ``W_{t+1}`` was changed
at check 6a. A transformers decoder step is verified the same way through ``DecoderReplay``:
its operands equal the prover's bit for bit, a product forged together with its claimed
operands is caught at check 5, and a forged glue-weight update at check 6b.
"""

from __future__ import annotations

import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

WIDTHS = (48, 96, 80, 24)


def _prove(seed=0, n_s=32, perturb=None, widths=WIDTHS):
    from verification.computation.instances.mlp import (MLPComputation, init_weights,
                                                        synthetic_dataset)
    from verification.prover.step import commit, prove_step
    c = MLPComputation(widths, n_s=n_s, eta=0.05)
    model = c.build_model().cuda()
    w0 = init_weights(widths, seed, "cuda")
    records = synthetic_dataset(widths, n_s, seed + 7)
    step = prove_step(c, model, w0, records, perturb=perturb)
    return c, step, commit(c, step)


def _oracle_root(c, leaves):
    hashes = []
    for i, obj in enumerate(leaves):
        if i < c.n_s:
            hashes.append(O.tensor_leaf_hash(0x04, obj.cpu()))
        else:
            tag = O.TAG_PRODUCT if c.n_s + c.n_w <= i < c.n_s + c.n_w + c.M else O.TAG_WEIGHT
            hashes.append(O.tensor_leaf_hash(tag, obj.cpu()))
    return O.merkle_root(hashes)


def test_products_stay_in_hbm_and_commit_matches_the_oracle(lib):
    c, step, tree = _prove(seed=1)
    assert step.capture["on_device"] and step.capture["products"] == c.M
    assert all(p.is_cuda for p in step.products)
    assert all(w.is_cuda for w in step.w_next.values())
    assert tree.root == _oracle_root(c, step.leaves())


def test_honest_step_accepts_with_the_replay(lib):
    from verification.transcript.store import InMemoryStore
    from conftest import started_verifier
    c, step, tree = _prove(seed=2)
    v = started_verifier(c, step.leaves(), k=2)
    assert v.verify_step(1, InMemoryStore(step.leaves(), tree)) is None
    assert [s.m for s in v.stats[1].products] == [p.m for p in c.products]
    assert v.stats[1].max_normalized() <= 8.0


def test_device_step_verifier_with_the_replay(lib):
    from verification.computation.instances.mlp import MLPReplay
    from verification.verifier.step import DeviceStepVerifier
    c, step, tree = _prove(seed=3)
    replay = MLPReplay(c, step.leaves())
    out = DeviceStepVerifier(c, step.leaves(), lambda s: replay.operands(s.m), k=2).run(
        tree.root)
    assert out.check is None, out.detail
    assert out.root == tree.root and out.first_fail == c.M


def test_perturbed_product_rejects_at_check_5(lib):
    from verification.transcript.store import InMemoryStore
    from conftest import started_verifier
    m = 2  # Y_2, a forward product: check 6a does not read it
    c, step, tree = _prove(seed=4, perturb={m: lambda p: p.index_add_(
        0, torch.tensor([3], device=p.device), torch.full_like(p[:1], 0.25))})
    rej = started_verifier(c, step.leaves(), k=2).verify_step(
        1, InMemoryStore(step.leaves(), tree))
    assert rej is not None and (rej.check_id, rej.kind) == ("5", "failed"), rej
    assert rej.detail.startswith(f"P_{m} (Y_2)")


def test_changed_update_rejects_at_check_6a(lib):
    from verification.commitment.leaves import commit_leaves_device
    from verification.transcript.store import InMemoryStore
    from conftest import started_verifier
    c, step, _ = _prove(seed=5)
    leaves = step.leaves()
    i = c.w_next_index(c.weight(2))
    leaves[i] = leaves[i].clone()
    leaves[i][0, 0] += 1e-2
    tree = commit_leaves_device(c, leaves)
    rej = started_verifier(c, leaves, k=2).verify_step(1, InMemoryStore(leaves, tree))
    assert rej is not None and rej.check_id == "6a", rej


def test_stored_mlp_step_verifies_from_disk(lib, tmp_path):
    from verification.transcript.loader import ResidentStore, load_step
    from verification.transcript.store import DiskStore
    from conftest import started_verifier
    c, step, tree = _prove(seed=6)
    disk = DiskStore.write(tmp_path / "step", c, step.leaves(), tree)
    res = load_step(disk, c.n_leaves)
    assert res.fallback == 0  # records are plain tensor leaves here
    for store in (disk, ResidentStore(disk, res)):
        assert started_verifier(c, step.leaves(), k=2).verify_step(1, store) is None


def _decoder_prove(seed=0, qkv_bias=True, n_kv=2, perturb=None, dtype=torch.float32,
                   c=None):
    from setup.records import Record
    from verification.computation.instances.decoder import DecoderComputation
    from verification.computation.interface import snapshot_weights
    from verification.prover.step import commit, prove_step
    if c is None:
        c = DecoderComputation(L=2, d=128, d_f=256, n_h=4, n_kv=n_kv, n_v=320, n_s=2, n=64,
                               qkv_bias=qkv_bias, compute_dtype=dtype)
    torch.manual_seed(seed)
    with torch.device("cuda"):
        model = c.build_model()
    w0 = snapshot_weights(c, model)
    g = torch.Generator().manual_seed(seed + 1)
    records = []
    for _ in range(c.n_s):
        ids = torch.randint(0, c.n_v, (c.n,), generator=g, dtype=torch.int32)
        records.append(Record(ids, torch.roll(ids, -1), torch.ones(c.n, dtype=torch.int32)))
    step = prove_step(c, model, w0, records, keep_operands=True, perturb=perturb)
    return c, step, commit(c, step)


def _decoder_oracle_root(c, leaves):
    hashes = []
    for i, obj in enumerate(leaves):
        if i < c.n_s:
            hashes.append(O.hash_leaf(O.encode_record(obj.ids, obj.targets, obj.mask)))
        else:
            tag = O.TAG_PRODUCT if c.n_s + c.n_w <= i < c.n_s + c.n_w + c.M else O.TAG_WEIGHT
            hashes.append(O.tensor_leaf_hash(tag, obj.cpu()))
    return O.merkle_root(hashes)


@pytest.mark.parametrize("qkv_bias,n_kv,dtype", [(True, 2, torch.float32),
                                                  (False, 4, torch.float32),
                                                  (True, 2, torch.bfloat16),
                                                  (False, 4, torch.bfloat16)])
def test_real_decoder_step_commits_and_verifies(lib, qkv_bias, n_kv, dtype):
    """A transformers Qwen2/Llama training step proved on the GPU, in fp32 or in bf16 under
    autocast over fp32 masters: the products stay in HBM, the device commit equals the CPU
    oracle's root, and the verifier accepts the step from the committed leaves alone (the
    decoder replay serves check 5's operands and check 6b's glue gradients) through the
    check-level API and the device step alike; the replay's operands are the prover's, bit for
    bit."""
    from conftest import started_verifier
    from verification.computation.instances.decoder import DecoderReplay
    from verification.transcript.store import InMemoryStore
    from verification.verifier.step import DeviceStepVerifier
    c, step, tree = _decoder_prove(seed=7, qkv_bias=qkv_bias, n_kv=n_kv, dtype=dtype)
    assert all(p.dtype == dtype for p in step.products)
    assert step.capture["on_device"]
    assert tree.root == _decoder_oracle_root(c, step.leaves())
    v = started_verifier(c, step.leaves(), k=2)
    assert v.verify_step(1, InMemoryStore(step.leaves(), tree)) is None
    assert len(v.stats[1].products) == c.M and not v.stats[1].operands_from_prover
    assert [t.weight for t in v.stats[1].tensors if t.check_id == "6b"] == \
        list(c.glue_gradient_weights)
    replay = DecoderReplay(c, step.leaves())
    for spec in c.products[::7]:
        assert all(torch.equal(x, y) for x, y in zip(replay.operands(spec.m),
                                                     step.operands[spec.m])), spec.name
    out = DeviceStepVerifier(c, step.leaves(), lambda s: replay.operands(s.m), k=2).run(tree.root)
    assert out.check is None and out.root == tree.root, out.detail


@pytest.mark.parametrize("tied,dtype", [(True, torch.bfloat16), (False, torch.bfloat16),
                                        (False, torch.float32)])
def test_head_blocks_step_commits_and_verifies(lib, tied, dtype):
    """The output layer in two row blocks (reference decoder.py:211-229, 740-770) proved on
    the GPU: the device commit equals the oracle's root; the verifier accepts the step from
    the committed leaves alone through the check-level API and the device step, the replay
    serving every head block's operands equal to the prover's; an untied W_out is checked at
    6a over its two G_head blocks, a tied embedding at 6b."""
    from conftest import started_verifier
    from verification.computation.instances.decoder import DecoderComputation, DecoderReplay
    from verification.transcript.store import InMemoryStore
    from verification.verifier.step import DeviceStepVerifier
    c = DecoderComputation(L=2, d=128, d_f=256, n_h=4, n_kv=2, n_v=320, n_s=4, n=64,
                           qkv_bias=True, compute_dtype=dtype, head_blocks=2, tied=tied)
    c, step, tree = _decoder_prove(seed=12, c=c)
    assert tree.root == _decoder_oracle_root(c, step.leaves())
    v = started_verifier(c, step.leaves(), k=2)
    assert v.verify_step(1, InMemoryStore(step.leaves(), tree)) is None
    checked = {t.weight: t.check_id for t in v.stats[1].tensors}
    assert checked[c.w_out] == ("6b" if tied else "6a")
    replay = DecoderReplay(c, step.leaves())
    for spec in c.products:
        if spec.weight == c.w_out:
            assert all(torch.equal(x, y) for x, y in zip(replay.operands(spec.m),
                                                         step.operands[spec.m])), spec.name
    out = DeviceStepVerifier(c, step.leaves(), lambda s: replay.operands(s.m), k=2).run(tree.root)
    assert out.check is None and out.root == tree.root, out.detail


def test_head_block_forgeries_reject(lib):
    """Two head blocks: a changed G_E_head[1] of a tied head rejects at check 5 at that
    product (the checks run 6a before 5, and the tied embedding's update is check 6b's), and
    an untied W_out update that is not W_t − η·(G_head[0] + G_head[1]) at check 6a."""
    from conftest import started_verifier
    from verification.commitment.leaves import commit_leaves_device
    from verification.computation.instances.decoder import DecoderComputation
    from verification.transcript.store import InMemoryStore

    def made(tied):
        return DecoderComputation(L=2, d=128, d_f=256, n_h=4, n_kv=2, n_v=320, n_s=4, n=64,
                                  qkv_bias=True, compute_dtype=torch.bfloat16, head_blocks=2,
                                  tied=tied)
    spec = next(s for s in made(True).products if s.name == "G_E_head[1]")
    c, step, tree = _decoder_prove(seed=13, c=made(True), perturb={
        spec.m: lambda p: p.index_add_(0, torch.tensor([9], device=p.device),
                                       torch.full_like(p[:1], 4.0))})
    rej = started_verifier(c, step.leaves(), k=2).verify_step(
        1, InMemoryStore(step.leaves(), tree))
    assert rej is not None and (rej.check_id, rej.kind) == ("5", "failed"), rej
    assert rej.detail.startswith(f"P_{spec.m} (G_E_head[1])")
    c, step, _ = _decoder_prove(seed=13, c=made(False))
    leaves = step.leaves()
    i = c.w_next_index(c.w_out)
    leaves[i] = leaves[i].clone()
    leaves[i][5, 7] += 1e-2
    rej = started_verifier(c, leaves, k=2).verify_step(
        1, InMemoryStore(leaves, commit_leaves_device(c, leaves)))
    assert rej is not None and rej.check_id == "6a" and c.w_out in rej.detail, rej


def test_real_decoder_step_with_a_changed_member_rejects_at_check_5(lib):
    from conftest import started_verifier
    from verification.transcript.store import InMemoryStore
    c0, _, _ = _decoder_prove(seed=8)
    spec = next(s for s in c0.products if s.name == "L2.O[1,3]")
    c, step, tree = _decoder_prove(seed=8, perturb={spec.m: lambda p: p.index_add_(
        0, torch.tensor([5], device=p.device), torch.full_like(p[:1], 0.5))})
    rej = started_verifier(c, step.leaves(), k=2).verify_step(
        1, InMemoryStore(step.leaves(), tree))
    assert rej is not None and (rej.check_id, rej.kind) == ("5", "failed"), rej
    assert rej.detail.startswith(f"P_{spec.m} (L2.O[1,3])")


def test_forged_operands_are_caught_by_the_replay(lib):
    """A prover that commits ``P' = A'·B`` for a forged input ``A'`` has a product consistent
    with the operands it would claim: trusting those operands accepts the step, the replay of
    the committed leaves rejects it at that product."""
    from conftest import started_verifier
    from verification.commitment.leaves import commit_leaves_device
    from verification.prover.synthetic import CapturedReplay
    from verification.transcript.store import InMemoryStore
    c, step, _ = _decoder_prove(seed=9)
    spec = next(s for s in c.products if s.name == "L2.Y_gate")
    a, b = step.operands[spec.m]
    a_forged = a.clone()
    a_forged[7] += 0.25
    leaves = step.leaves()
    leaves[c.product_index(spec.m)] = torch.mm(a_forged, b)
    tree = commit_leaves_device(c, leaves)
    claimed = {m: ((a_forged, b) if m == spec.m else ops) for m, ops in step.operands.items()}
    c.use_operands(CapturedReplay(claimed))
    trusted = started_verifier(c, leaves, k=2).verify_step(1, InMemoryStore(leaves, tree))
    c.use_operands(None)
    rej = started_verifier(c, leaves, k=2).verify_step(1, InMemoryStore(leaves, tree))
    assert rej is not None and (rej.check_id, rej.kind) == ("5", "failed"), rej
    assert rej.detail.startswith(f"P_{spec.m} (L2.Y_gate)")
    # with the prover's operands every check passes (6b, which needs the replay's glue, is
    # not run for them): the forgery is caught only by the replay
    assert trusted is None


def test_forged_glue_update_rejects_at_check_6b(lib):
    from conftest import started_verifier
    from verification.commitment.leaves import commit_leaves_device
    from verification.transcript.store import InMemoryStore
    c, step, _ = _decoder_prove(seed=10)
    name = next(n for n in c.glue_gradient_weights if "post_attention_layernorm" in n)
    leaves = step.leaves()
    i = c.w_next_index(name)
    leaves[i] = leaves[i].clone()
    leaves[i][3] += 1e-3
    rej = started_verifier(c, leaves, k=2).verify_step(
        1, InMemoryStore(leaves, commit_leaves_device(c, leaves)))
    assert rej is not None and (rej.check_id, rej.kind) == ("6b", "failed"), rej
    assert rej.detail.startswith(f"{name}: entry 3 has |R| = ")


def test_c1_real_smollm2_step_proves_commits_and_verifies(lib):
    """BASELINE config 0 as specified: a SmolLM2-135M-shaped Llama (30 layers, d 576, 9/3
    heads of dim 64, MLP 1536, vocab 49152, tied; random-init fp32), one plain-SGD step at lr
    1e-4 on 4 x 256 random token ids, every matmul captured, the transcript committed (root
    checked against the CPU oracle) and verified with k = 1."""
    from setup.records import Record
    from verification.computation.instances.decoder import smollm2_135m
    from verification.computation.interface import snapshot_weights
    from verification.prover.step import commit, prove_step
    from verification.transcript.store import InMemoryStore
    from conftest import started_verifier
    c = smollm2_135m()
    torch.manual_seed(0)
    with torch.device("cuda"):
        model = c.build_model()
    w0 = snapshot_weights(c, model)
    g = torch.Generator().manual_seed(0)
    records = []
    for _ in range(c.n_s):
        ids = torch.randint(0, c.n_v, (c.n,), generator=g, dtype=torch.int32)
        records.append(Record(ids, torch.roll(ids, -1), torch.ones(c.n, dtype=torch.int32)))
    step = prove_step(c, model, w0, records, keep_operands=True)
    assert len(step.products) == c.M == 7113
    tree = commit(c, step)
    assert tree.root == _decoder_oracle_root(c, step.leaves())
    v = started_verifier(c, step.leaves(), k=1)
    assert v.verify_step(1, InMemoryStore(step.leaves(), tree)) is None
    assert len(v.stats[1].products) == c.M and v.stats[1].max_normalized() <= 8.0


def test_bf16_decoder_at_c4_dimensions_proves_and_verifies_from_its_leaves(lib):
    """Two layers of the Qwen2-1.5B shape (d 1536, 12/2 heads of 128, MLP 8960, vocab 151,936,
    4 x 2048 tokens) in bf16 under autocast over fp32 masters: the device commit equals the
    CPU oracle's root over every leaf; the replay of the committed leaves serves every
    product's operands equal to the prover's bit for bit; the honest step accepts with no
    prover operands trusted (checks 6a and 6b included); and a product forged together with
    the forged operand it was made from is caught at check 5 by the replay, though the
    prover's operands would pass it."""
    import sys
    from conftest import started_verifier
    from test_fullsize_gpu import _oracle_digests
    from verification.commitment.leaves import commit_leaves_device
    from verification.computation.instances.decoder import DecoderComputation, DecoderReplay
    from verification.prover.synthetic import CapturedReplay
    from verification.transcript.store import InMemoryStore

    def say(msg):
        print(f"[c4-bf16] {msg}", file=sys.__stderr__, flush=True)

    c = DecoderComputation(L=2, d=1536, d_f=8960, n_h=12, n_kv=2, n_v=151936, n_s=4, n=2048,
                           d_h=128, tied=True, qkv_bias=True, compute_dtype=torch.bfloat16)
    c, step, tree = _decoder_prove(seed=11, c=c)
    say(f"proved and committed: {c.M} products")
    assert all(p.dtype == torch.bfloat16 and p.is_cuda for p in step.products)
    assert tree.root == O.merkle_root(_oracle_digests(c, step.leaves()))
    say("root equals the oracle's")
    replay = DecoderReplay(c, step.leaves())
    for spec in c.products:
        got, want = replay.operands(spec.m), step.operands[spec.m]
        assert all(x.dtype == torch.bfloat16 for x in got), spec.name
        assert all(torch.equal(x, y) for x, y in zip(got, want)), spec.name
    say("replay operands equal the prover's")
    del replay
    v = started_verifier(c, step.leaves(), k=4)
    assert not v.trust_prover_operands
    assert v.verify_step(1, InMemoryStore(step.leaves(), tree)) is None
    assert not v.stats[1].operands_from_prover and len(v.stats[1].products) == c.M
    assert {t.check_id for t in v.stats[1].tensors} == {"6a", "6b"}
    say("honest step accepted")
    v.close()
    spec = next(s for s in c.products if s.name == "L2.Y_gate")
    a, b = step.operands[spec.m]
    a_forged = a.clone()
    # one row of the gate's input shifted by 16: at these widths a bf16 product's band unit
    # (ε_in = 2⁻⁸ on ‖P‖_F ≈ 7e3) hides a shift of 0.25, so the forgery must be larger
    a_forged[7] += 16.0
    leaves = step.leaves()
    leaves[c.product_index(spec.m)] = torch.mm(a_forged, b.contiguous())
    forged_tree = commit_leaves_device(c, leaves)
    c.use_operands(CapturedReplay({**step.operands, spec.m: (a_forged, b)}))
    v = started_verifier(c, leaves, k=4)
    assert v.trust_prover_operands
    assert v.verify_step(1, InMemoryStore(leaves, forged_tree)) is None
    v.close()
    c.use_operands(None)
    v = started_verifier(c, leaves, k=4)
    assert not v.trust_prover_operands
    rej = v.verify_step(1, InMemoryStore(leaves, forged_tree))
    v.close()
    assert rej is not None and (rej.check_id, rej.kind) == ("5", "failed"), rej
    assert rej.detail.startswith(f"P_{spec.m} (L2.Y_gate)")
    say("forged operand caught at check 5")
