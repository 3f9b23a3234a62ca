"""The prover side on the host: the matmul capture's recording rules (reference
tests/verification/prover/test_capture.py), the MLP computation's inventory, labeling and SGD
step (reference instances/mlp.py, prover/step.py), and the MLP replay's operands, which must
reproduce every committed product bit for bit on the same device.
"""

from __future__ import annotations

import pytest
import torch

from verification.computation.instances.mlp import (MLPComputation, MLPReplay, init_weights,
                                                    synthetic_dataset)
from verification.computation.interface import ProductKind
from verification.computation.matmul_ops import HANDLED_OPS, REJECTED_OPS, param_storage_map
from verification.prover.capture import (BiasedMatmulError, MatmulCapture,
                                         MutatedCaptureError, PhaseError,
                                         UnsupportedMatmulError)
from verification.prover.step import prove_step

WIDTHS = (6, 9, 7, 5)


def test_op_lists_name_real_aten_ops():
    missing = [n for n in sorted(HANDLED_OPS | REJECTED_OPS)
               if not hasattr(torch.ops.aten, n)]
    # a few names exist only on some builds (MPS, CUDA-only kernels); the rest must resolve
    assert len(missing) < 15, missing
    assert not HANDLED_OPS & REJECTED_OPS


def test_capture_records_products_with_their_operands():
    a, b = torch.randn(4, 3), torch.randn(3, 5)
    bias = torch.randn(5)
    x, y = torch.randn(2, 4, 3), torch.randn(2, 3, 6)
    cap = MatmulCapture()
    with cap, cap.phase("forward"):
        p1 = torch.mm(a, b)
        p2 = torch.addmm(bias, a, b)                        # the bias rule: a vector added once
        p3 = torch.bmm(x, y)
        p4 = torch.addmm(torch.zeros(4, 5), a, b)           # an inert bias
        p5 = torch.baddbmm(torch.zeros(2, 4, 6), x, y, beta=0)
    assert [r.op for r in cap.records] == ["aten.mm.default", "aten.addmm.default",
                                           "aten.bmm.default", "aten.addmm.default",
                                           "aten.baddbmm.default"]
    assert all(r.out is p for r, p in zip(cap.records, (p1, p2, p3, p4, p5)))
    assert cap.records[1].bias is bias and cap.records[0].bias is None
    assert cap.records[2].batch == 2 and cap.n_products == 1 + 1 + 2 + 1 + 2
    assert [m[2].shape for m in cap.records[2].members()] == [(4, 6), (4, 6)]
    assert all(r.q == 3 for r in cap.records) and not cap.glue_outer
    s = cap.summary()
    assert s["calls"] == 5 and s["products"] == 7 and s["products_per_phase"] == {
        "forward": 7}
    assert s["calls_per_op"]["forward:aten.addmm.default"] == 2 and s["q_range"] == (3, 3)
    assert s["outer_calls"] == 0 and s["product_bytes"] == 4 * (20 + 20 + 48 + 20 + 48)


def test_capture_rules_refuse_what_the_inventory_cannot_hold():
    a, b = torch.randn(4, 3), torch.randn(3, 5)
    cap = MatmulCapture()
    with cap:
        with pytest.raises(PhaseError):
            torch.mm(a, b)                                  # outside a phase
        with cap.phase("forward"):
            with pytest.raises(PhaseError):
                with cap.phase("backward"):
                    pass
            with pytest.raises(BiasedMatmulError):
                torch.addmm(torch.ones(4, 5), a, b)         # a matrix bias
            with pytest.raises(BiasedMatmulError):
                torch.addmm(torch.ones(5), a, b, alpha=2)
            with pytest.raises(BiasedMatmulError):
                torch.baddbmm(torch.ones(5), a[None], b[None])  # a batched product's bias
            with pytest.raises(UnsupportedMatmulError):
                torch.mv(a, torch.randn(3))
            with pytest.raises(UnsupportedMatmulError):
                torch.ops.aten.mm.out(a, b, out=torch.empty(4, 5))
            torch.mm(torch.randn(4, 1), torch.randn(1, 5))  # q = 1: an outer product, glue
    with pytest.raises(PhaseError):
        with cap.phase("sideways"):
            pass
    assert len(cap.glue_outer) == 1 and not cap.records


def test_capture_tracks_producers_parameter_copies_and_mutation():
    lin = torch.nn.Linear(3, 4, bias=False)
    names = param_storage_map(lin)
    x = torch.randn(5, 3)
    cap = MatmulCapture(param_names=names)
    with cap:
        with cap.phase("forward"):
            y = lin(x)
            w16 = lin.weight.to(torch.float64)              # a copy of a parameter
            z = torch.mm(y, torch.randn(4, 2))
            torch.mm(x.double(), w16.t())
    fwd, second, third = cap.records
    assert fwd.b_info.param_name == "weight"
    assert second.a_info.producer_index == fwd.index       # z's A is y, fwd's output
    assert third.b_info.param_copy == "weight" and third.b_info.param_name is None
    assert any(c.param == "weight" for c in cap.copies)
    cap.assert_unmodified()
    z.add_(1.0)
    with pytest.raises(MutatedCaptureError):
        cap.assert_unmodified()
    cap.release_operands()
    assert all(r.a is None and r.b is None for r in cap.records)


def test_capture_refusals_outside_a_phase():
    a, b = torch.randn(4, 3), torch.randn(3, 5)
    cap = MatmulCapture()
    with cap:
        # a refused matmul-like op and another overload of a handled op are refused anywhere
        with pytest.raises(UnsupportedMatmulError):
            torch.mv(a, torch.randn(3))
        with pytest.raises(UnsupportedMatmulError):
            torch.ops.aten.bmm.out(a[None], b[None], out=torch.empty(1, 4, 5))
        # a handled op, a copy and an ordinary op outside a phase: the first is refused, the
        # others run and leave nothing behind
        with pytest.raises(PhaseError):
            torch.mm(a, b)
        a.to(torch.float64)
        torch.relu(a)
        with cap.phase("backward"):
            torch.mm(a, b)
            w = a.to(torch.float64)                          # a copy of no parameter
    assert [r.phase for r in cap.records] == ["backward"] and len(cap.copies) == 1
    assert cap.copies[0].param is None and cap.param_of(w) is None


def test_capture_refuses_foreign_ops_only_inside_a_phase():
    lib = torch.library.Library("potstest", "DEF")
    lib.define("twice(Tensor x) -> Tensor")
    lib.impl("twice", lambda x: x * 2, "CompositeExplicitAutograd")
    x = torch.randn(3)
    cap = MatmulCapture()
    with cap:
        torch.ops.potstest.twice(x)                          # outside a phase: runs
        with cap.phase("forward"):
            with pytest.raises(UnsupportedMatmulError, match="outside aten and prims"):
                torch.ops.potstest.twice(x)


def test_capture_watch_names_each_moved_role_and_release_keeps_outputs():
    a, b = torch.randn(4, 3), torch.randn(3, 5)
    cap = MatmulCapture()
    with cap, cap.phase("forward"):
        p = torch.mm(a, b)
        torch.mm(p, torch.randn(5, 2))
    a.mul_(2)
    p.add_(1)
    with pytest.raises(MutatedCaptureError) as e:
        cap.assert_unmodified()
    msg = str(e.value)
    assert "#0 aten.mm.default (forward): a, out" in msg and "#1 aten.mm.default (forward): a" \
        in msg
    cap.release_operands()
    with pytest.raises(MutatedCaptureError):                 # outputs are still watched
        cap.assert_unmodified()
    assert cap.records[0].out is p and cap.records[0].a is None
    with pytest.raises(Exception, match="released"):
        list(cap.records[0].members())


def test_capture_parameter_copies_are_released():
    lin = torch.nn.Linear(3, 4, bias=False)
    cap = MatmulCapture(param_names=param_storage_map(lin))
    with cap, cap.phase("forward"):
        w64 = lin.weight.to(torch.float64)
        ww = w64.to(torch.float32)                          # a copy of the copy
    assert cap.param_of(w64) == "weight" and cap.param_of(ww) == "weight"
    assert cap.param_of(lin.weight) == "weight"
    assert [c.param for c in cap.copies] == ["weight", "weight"]
    assert cap.summary()["parameter_copies"] == 2
    cap.release_operands()
    assert cap.param_of(w64) is None and cap.param_of(lin.weight) == "weight"


def test_mlp_inventory_matches_the_reference_layout():
    c = MLPComputation(WIDTHS, n_s=4, eta=0.05)
    assert c.M == 3 * c.L - 1 == 8
    assert [p.name for p in c.products] == ["Y_1", "Y_2", "Y_3", "dX_3", "G_3", "dX_2", "G_2",
                                            "G_1"]
    g3 = c.product(c.m_of("G_3"))
    assert (g3.kind, g3.a_shape, g3.b_shape) == (ProductKind.WEIGHT_GRAD, (5, 4), (4, 7))
    assert c.linear_weights == {"layers.0.weight": (8,), "layers.1.weight": (7,),
                                "layers.2.weight": (5,)}
    assert c.n_leaves == 4 + 2 * 3 + 8
    with pytest.raises(ValueError):
        MLPComputation(WIDTHS, n_s=1, eta=0.05)
    with pytest.raises(ValueError):
        c.encode_record(torch.zeros(10))


def _step(seed=0, n_s=4, perturb=None):
    c = MLPComputation(WIDTHS, n_s=n_s, eta=0.05)
    model = c.build_model()
    w0 = init_weights(WIDTHS, seed)
    records = synthetic_dataset(WIDTHS, n_s, seed + 7)
    return c, w0, prove_step(c, model, w0, records, perturb=perturb), model


def test_prove_step_labels_products_and_steps_sgd():
    c, w0, step, model = _step()
    assert len(step.leaves()) == c.n_leaves
    x1, targets = c.assemble(step.records)
    ws = [w0[n] for n in c.weight_names]
    y1 = x1 @ ws[0].t()
    assert torch.allclose(step.products[c.m_of("Y_1") - 1], y1, rtol=1e-6, atol=1e-6)
    y2 = torch.tanh(y1) @ ws[1].t()
    assert torch.allclose(step.products[c.m_of("Y_2") - 1], y2, rtol=1e-5, atol=1e-6)
    # W_{t+1} = W_t − η·G_ℓ, G_ℓ the committed weight-gradient product
    for l in range(1, c.L + 1):
        g = step.products[c.m_of(f"G_{l}") - 1]
        assert torch.allclose(step.w_next[c.weight(l)], w0[c.weight(l)] - c.eta * g,
                              rtol=0, atol=1e-7)
    assert step.capture["products"] == c.M
    step.assert_unmodified()
    step.products[0].add_(1.0)
    with pytest.raises(MutatedCaptureError):
        step.assert_unmodified()


def test_prove_step_perturbation_changes_only_the_committed_leaf():
    m = 2
    c, _, honest, _ = _step()
    _, _, cheat, _ = _step(perturb={m: lambda p: p + 1.0})
    assert torch.equal(cheat.products[m - 1], honest.products[m - 1] + 1.0)
    for k in range(c.M):
        if k != m - 1:
            assert torch.equal(cheat.products[k], honest.products[k])


def test_replay_operands_reproduce_every_product():
    c, _, step, _ = _step(seed=3)
    replay = MLPReplay(c, step.leaves(), device="cpu")
    for spec in c.products:
        a, b = replay.operands(spec.m)
        assert (tuple(a.shape), tuple(b.shape)) == (spec.a_shape, spec.b_shape)
        assert torch.equal(torch.mm(a, b), step.products[spec.m - 1]), spec.name
    assert replay.glue_gradients() == {}
    # any order gives the same operands
    again = MLPReplay(c, step.leaves(), device="cpu")
    for spec in reversed(c.products):
        a, b = again.operands(spec.m)
        assert torch.equal(torch.mm(a, b), step.products[spec.m - 1]), spec.name


def _decoder_step(qkv_bias=True, n_kv=2, dtype=torch.float32, head_blocks=1, tied=True):
    from setup.records import Record
    from verification.computation.instances.decoder import DecoderComputation
    from verification.computation.interface import snapshot_weights
    c = DecoderComputation(L=2, d=64, d_f=128, n_h=4, n_kv=n_kv, n_v=160, n_s=2, n=16,
                           qkv_bias=qkv_bias, compute_dtype=dtype, head_blocks=head_blocks,
                           tied=tied)
    torch.manual_seed(0)
    model = c.build_model()
    w0 = snapshot_weights(c, model)
    g = torch.Generator().manual_seed(1)
    records = []
    for _ in range(c.n_s):
        ids = torch.randint(0, c.n_v, (c.n,), generator=g, dtype=torch.int32)
        records.append(Record(ids, torch.roll(ids, -1), torch.ones(c.n, dtype=torch.int32)))
    return c, w0, prove_step(c, model, w0, records, keep_operands=True)


DECODERS = [(True, 2, torch.float32), (False, 4, torch.float32), (True, 2, torch.bfloat16),
            (False, 4, torch.bfloat16)]


@pytest.mark.parametrize("qkv_bias,n_kv,dtype", DECODERS)
def test_decoder_labeling_fills_every_slot_with_its_own_product(qkv_bias, n_kv, dtype):
    """A transformers Qwen2 (biased q/k/v, grouped KV heads) or Llama step under the capture,
    in fp32 or in bf16 under autocast over fp32 masters: every declared slot is filled with a
    product of the compute dtype, and each product equals its captured operands' product
    (bit for bit for a plain fp32 product; the biased linears within rounding, bf16 products
    within one bf16 rounding of the fp32 sum)."""
    c, w0, step = _decoder_step(qkv_bias, n_kv, dtype)
    assert len(step.products) == c.M and step.capture["outer_calls"] == 1
    assert all(w.dtype == torch.float32 for w in step.w_next.values())
    for spec in c.products:
        a, b = step.operands[spec.m]
        p = step.products[spec.m - 1]
        assert p.dtype == dtype and a.dtype == dtype and b.dtype == dtype, spec.name
        assert (tuple(a.shape), tuple(b.shape)) == (spec.a_shape, spec.b_shape), spec.name
        q = torch.mm(a.float(), b.float())
        if spec.bias is not None:
            q = q + w0[spec.bias].to(dtype).float()
        if dtype == torch.bfloat16:
            scale = torch.mm(a.float().abs(), b.float().abs()) + 1e-30
            assert ((q - p.float()).abs() <= 2.0**-8 * scale + 1e-6).all(), spec.name
        elif spec.bias is not None:
            assert torch.allclose(q, p, rtol=1e-5, atol=1e-6), spec.name
        else:
            assert torch.equal(q, p), spec.name
    # a linear weight's update is its committed weight gradient's SGD step
    name = c.w(1, "up")
    g = step.products[c.product_index(c.linear_weights[name][0]) - c.n_s - c.n_w]
    assert torch.allclose(step.w_next[name], w0[name] - c.eta * g.float(), rtol=0, atol=1e-7)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decoder_batched_products_never_take_a_transposed_right_operand(dtype):
    """Every batched product of a decoder step, forward and backward, receives a contiguous
    right operand (bf16 batched products with a transposed right operand are kept off this
    pool's GPUs), and the left operands that are transposed views share storage with another
    product's left operand (dV with O, dK with dQ)."""
    from verification.computation.instances.decoder import DecoderComputation
    from verification.computation.matmul_ops import param_storage_map
    c = DecoderComputation(L=2, d=64, d_f=128, n_h=4, n_kv=2, n_v=160, n_s=2, n=16,
                           qkv_bias=True, compute_dtype=dtype)
    torch.manual_seed(0)
    model = c.build_model()
    from setup.records import Record
    ids = torch.randint(0, c.n_v, (c.n,), dtype=torch.int32)
    records = [Record(ids, torch.roll(ids, -1), torch.ones(c.n, dtype=torch.int32))] * c.n_s
    cap = MatmulCapture(param_names=param_storage_map(model))
    with cap:
        c.forward_backward(model, records, cap.phase)
    batched = [r for r in cap.records if r.batch is not None]
    assert len(batched) == 6 * c.L
    assert all(r.b.is_contiguous() for r in batched)
    assert all(r.a.dtype == dtype and r.b.dtype == dtype for r in batched)
    lefts = {r.a.untyped_storage().data_ptr() for r in batched if r.a.is_contiguous()}
    views = [r for r in batched if not r.a.is_contiguous()]
    assert len(views) == 2 * c.L and all(r.a.untyped_storage().data_ptr() in lefts
                                         for r in views)


def test_reference_inventory_literals():
    """The reference's declaration numbers (tests/verification/computation/test_decoder.py
    :167-184 at SmolLM2-135M, 4×128 tokens; test_sizing.py:45-48 and test_decoder.py:163-165
    for the product count)."""
    import math
    from collections import Counter

    from verification.computation.instances.decoder import matmul_count_decoder, smollm2_135m
    from verification.computation.interface import ProductKind as K
    c = smollm2_135m(n_s=4, n=128)
    assert (c.M, c.n_w, c.n_leaves) == (7113, 272, 7661)
    assert sum(math.prod(s) for s in c.weight_shapes.values()) == 134_515_008
    assert Counter(p.kind for p in c.products) == {K.FORWARD: 2371, K.INPUT_GRAD: 211,
                                                   K.WEIGHT_GRAD: 211, K.OPERAND_GRAD: 4320}
    linears = ("q", "k", "v", "o", "gate", "up", "down")
    q = {c.product_class(p): p.q for p in c.products}
    assert q == {"Y_q": 576, "Y_k": 576, "Y_v": 576, "Y_o": 576, "Y_gate": 576, "Y_up": 576,
                 "Y_down": 1536, "S": 64, "O": 128, "Lambda": 576,
                 "dF": 49152, "G_E_head": 512,
                 "dX_q": 576, "dX_k": 192, "dX_v": 192, "dX_o": 576, "dX_gate": 1536,
                 "dX_up": 1536, "dX_down": 576,
                 **{f"G_{x}": 512 for x in linears},
                 "dA": 64, "dV": 128, "dQ": 128, "dK": 128}
    per_member = c.L * c.n_s * c.n_h
    assert Counter(c.product_class(p) for p in c.products) == Counter(
        {**{f"{r}_{x}": c.L for r in ("Y", "dX", "G") for x in linears},
         **{r: per_member for r in ("S", "O", "dA", "dV", "dQ", "dK")},
         "Lambda": 1, "dF": 1, "G_E_head": 1})
    assert all(p.width == p.p_shape[1] for p in c.products)
    assert matmul_count_decoder(30, 4, 9) == 7_113
    assert matmul_count_decoder(30, 128, 9) == 207_993
    assert matmul_count_decoder(16, 128, 32) == 393_555


def test_decoder_bf16_runs_under_autocast_over_fp32_masters():
    """A bf16 decoder keeps fp32 master weights and computes its logits in bf16 under
    autocast (reference decoder.py:551-598); the loss itself is fp32."""
    from verification.computation.instances.decoder import DecoderComputation
    from setup.records import Record
    c = DecoderComputation(L=1, d=16, d_f=32, n_h=2, n_kv=1, n_v=40, n_s=1, n=8,
                           compute_dtype=torch.bfloat16)
    model = c.build_model()
    assert not model.training
    assert all(p.dtype == torch.float32 for p in model.parameters())
    ids = torch.arange(c.n, dtype=torch.int32)
    with c.autocast(torch.device("cpu")):
        logits = model(input_ids=ids[None].long()).logits
    assert logits.dtype == torch.bfloat16
    loss = c.loss(model, [Record(ids, ids, torch.ones(c.n, dtype=torch.int32))])
    assert loss.dtype == torch.float32 and torch.isfinite(loss)
    fp32 = DecoderComputation(L=1, d=16, d_f=32, n_h=2, n_kv=1, n_v=40, n_s=1, n=8)
    with fp32.autocast(torch.device("cpu")):
        assert fp32.build_model()(input_ids=ids[None].long()).logits.dtype == torch.float32


@pytest.mark.parametrize("qkv_bias,n_kv,dtype", DECODERS)
def test_decoder_replay_rebuilds_the_operands_from_the_leaves(qkv_bias, n_kv, dtype):
    """The verifier's replay (the committed leaves only, every product substituted by its
    leaf) gives every product the operands the prover's capture saw, bit for bit, and each
    glue weight (γ, biases, the tied embedding) the gradient SGD stepped with."""
    from verification.computation.instances.decoder import DecoderReplay
    c, w0, step = _decoder_step(qkv_bias, n_kv, dtype)
    leaves = step.leaves()
    replay = DecoderReplay(c, leaves, device="cpu")
    for spec in c.products:
        a, b = replay.operands(spec.m)
        ca, cb = step.operands[spec.m]
        assert torch.equal(a, ca) and torch.equal(b, cb), spec.name
    glue = replay.glue_gradients()
    assert set(glue) == set(c.glue_gradient_weights) and c.w_out in glue
    for name, g in glue.items():
        want = torch.add(leaves[c.w_t_index(name)], g, alpha=-c.eta)
        assert torch.equal(want, leaves[c.w_next_index(name)]), name
    # a second replay reuses the plan and gives the same operands
    again = DecoderReplay(c, leaves, device="cpu")
    m = c.products[len(c.products) // 2].m
    assert all(torch.equal(x, y) for x, y in zip(again.operands(m), replay.operands(m)))


@pytest.mark.parametrize("qkv_bias,n_kv,dtype", DECODERS)
def test_decoder_replay_serves_each_attention_call_as_one_group(qkv_bias, n_kv, dtype):
    """``operand_group`` over a batched call's members returns the call's whole operands (a
    view, no copy) equal to the members' operands stacked; a group it does not hold (a
    reordered or partial one) is stacked member by member."""
    from verification.computation.instances.decoder import DecoderReplay
    c, w0, step = _decoder_step(qkv_bias, n_kv, dtype)
    replay = DecoderReplay(c, step.leaves(), device="cpu")
    groups = [g for g in c.operand_groups if len(g) > 1]
    assert len(groups) == 6 * c.L  # S, O, dA, dV, dQ, dK per layer
    for g in groups:
        ms = [c.products[i].m for i in g]
        a, b = replay.operand_group(ms)
        pairs = [replay.operands(m) for m in ms]
        assert torch.equal(a, torch.stack([x for x, _ in pairs]))
        assert torch.equal(b, torch.stack([y for _, y in pairs]))
        assert a[0].data_ptr() == pairs[0][0].data_ptr()  # served where the call left it
    ms = [c.products[i].m for i in groups[0]]
    a, _ = replay.operand_group(ms[::-1])
    assert torch.equal(a, torch.stack([replay.operands(m)[0] for m in ms[::-1]]))
    assert a.data_ptr() != replay.operands(ms[-1])[0].data_ptr()


HEADS = [(True, torch.float32), (False, torch.float32), (True, torch.bfloat16),
         (False, torch.bfloat16)]


@pytest.mark.parametrize("tied,dtype", HEADS)
def test_head_blocks_fill_their_slots_and_chain_the_head_gradient(tied, dtype):
    """The output layer in two row blocks (reference decoder.py:211-229, 740-770): 3B head
    products, each block's Λ_b, dF_b and G_b in its own slot and equal to its captured
    operands' product; Λ_b's A is block b's rows of the features, so the blocks' Λ stack to
    the one-block step's Λ (the same weights and batch); the loss is the one-block loss; an
    untied W_out steps by its blocks' G_b widened to fp32 and added in block order."""
    from verification.computation.instances.decoder import matmul_count_decoder
    from verification.computation.interface import chain_gradient
    c, w0, step = _decoder_step(True, 2, dtype, head_blocks=2, tied=tied)
    one, _, whole = _decoder_step(True, 2, dtype, head_blocks=1, tied=tied)
    assert c.M == matmul_count_decoder(c.L, c.n_s, c.n_h, 2) == one.M + 3
    assert step.capture["outer_calls"] == 1
    names = [s.name for s in c.products]
    g_head = "G_E_head" if tied else "G_head"
    for b in range(2):
        assert {f"Lambda[{b}]", f"dF[{b}]", f"{g_head}[{b}]"} <= set(names)
    for spec in c.products:
        a, b = step.operands[spec.m]
        p = step.products[spec.m - 1]
        assert p.dtype == dtype and (tuple(a.shape), tuple(b.shape)) == (spec.a_shape,
                                                                           spec.b_shape)
        q = torch.mm(a.float(), b.float())
        if spec.bias is not None:
            q = q + w0[spec.bias].to(dtype).float()
        scale = torch.mm(a.float().abs(), b.float().abs()) + 1e-30
        tol = 2.0**-8 if dtype == torch.bfloat16 else 1e-5
        assert ((q - p.float()).abs() <= tol * scale + 1e-6).all(), spec.name
    lam = [step.products[names.index(f"Lambda[{b}]")] for b in range(2)]
    lam1 = whole.products[[s.name for s in one.products].index("Lambda")]
    tol = 2.0**-7 if dtype == torch.bfloat16 else 1e-5
    assert torch.allclose(torch.cat(lam).float(), lam1.float(), rtol=tol, atol=tol)
    assert step.loss == pytest.approx(whole.loss, rel=1e-5)
    if not tied:
        gs = [step.products[names.index(f"G_head[{b}]")] for b in range(2)]
        want = torch.add(w0[c.w_out], chain_gradient(gs, torch.float32), alpha=-c.eta)
        assert torch.equal(step.w_next[c.w_out], want)
        assert c.linear_weights[c.w_out] == tuple(
            c.products[names.index(f"G_head[{b}]")].m for b in range(2))


@pytest.mark.parametrize("tied,dtype", HEADS)
def test_head_blocks_replay_from_the_leaves(tied, dtype):
    """The replay of a two-block step gives every product, the head blocks' included, the
    operands the capture saw, bit for bit, and each glue weight (a tied embedding: its lookup
    gradient plus the blocks' committed G_E_head[b]) the gradient SGD stepped with."""
    from verification.computation.instances.decoder import DecoderReplay
    c, w0, step = _decoder_step(True, 2, dtype, head_blocks=2, tied=tied)
    leaves = step.leaves()
    replay = DecoderReplay(c, leaves, device="cpu")
    for spec in c.products:
        a, b = replay.operands(spec.m)
        ca, cb = step.operands[spec.m]
        assert torch.equal(a, ca) and torch.equal(b, cb), spec.name
    glue = replay.glue_gradients()
    assert set(glue) == set(c.glue_gradient_weights) and (c.w_out in glue) == tied
    for name, g in glue.items():
        want = torch.add(leaves[c.w_t_index(name)], g, alpha=-c.eta)
        assert torch.equal(want, leaves[c.w_next_index(name)]), name


def test_operand_groups_follow_the_batched_products():
    """Every product in exactly one group, groups in order of their first product; members of
    one layer's role together even where two roles interleave."""
    from verification.computation.instances.decoder import DecoderComputation
    c = DecoderComputation(L=2, d=64, d_f=128, n_h=4, n_kv=2, n_v=160, n_s=2, n=32)
    groups = c.operand_groups
    assert sorted(i for g in groups for i in g) == list(range(c.M))
    assert [g[0] for g in groups] == sorted(g[0] for g in groups)
    for g in groups:
        names = {c.products[i].name.split("[")[0] for i in g}
        assert len(names) == 1 and list(g) == sorted(g)
        if len(g) > 1:
            assert len(g) == c.n_s * c.n_h
    da = next(g for g in groups if c.products[g[0]].name.startswith("L2.dA"))
    assert da[1] - da[0] == 2  # dA and dV interleave in canonical order


def test_decoder_replay_follows_a_forged_product():
    """A forged forward product changes the glue downstream of it: the replay serves the
    operands the committed leaves imply, so the forged product itself no longer equals its
    operands' product, and later products' operands move with it."""
    from verification.computation.instances.decoder import DecoderReplay
    c, w0, step = _decoder_step(True, 2)
    leaves = step.leaves()
    spec = next(s for s in c.products if s.name == "L1.Y_up")
    i = c.product_index(spec.m)
    forged = list(leaves)
    forged[i] = leaves[i].clone()
    forged[i][3, 5] += 1.0
    replay = DecoderReplay(c, forged, device="cpu")
    a, b = replay.operands(spec.m)
    assert torch.equal(a, step.operands[spec.m][0])  # Y_up's own input is upstream
    assert not torch.equal(torch.mm(a, b) + 0, forged[i])
    down = next(s for s in c.products if s.name == "L1.Y_down")
    assert not torch.equal(replay.operands(down.m)[0], step.operands[down.m][0])
