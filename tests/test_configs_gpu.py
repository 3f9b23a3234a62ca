"""The benchmark configurations as parity cases on the GPU.

- C2, the fp32 single-matmul microbench (A 8192x4096, B 4096x4096, C = A·B, k = 1 and 8,
  leaves [A, B, C] with the product tag, challenges from their 3-leaf root): the root
  bit for bit, the row within the Freivalds tolerances, and the verdict of the honest and of
  the tampered C (one entry times 1 + 1e-2) equal to the oracle's. Per the reference's own
  band unit that tamper stays below τ, so parity means accepting it, as the reference does.
- C1 at its full size (SmolLM2-135M step, fp32, k = 1): the recomputed root equal to the
  oracle's over every leaf, the step accepted, and a sample of rows against the oracle.
- C5, the adversarial variant, scaled to two layers of C4's dimensions with a 4096-token
  vocabulary (k = 16, 5% of the products perturbed by 1 ± x, x log-uniform in [1e-6, 1]): the
  per-product verdicts equal to the oracle's for every perturbed product and a sample of
  honest ones. A product whose largest normalized residual lies within 0.1% of τ is reported
  instead of asserted: there the last bits of fp32 arithmetic decide the verdict, and the
  reference notes that those bits depend on operand layout, batch and platform
  (freivalds.py:56-64). A single-entry change of at most 100% of a bf16 entry stays inside a
  bf16 product's band at these shapes, so the reference accepts such products; parity means
  the same verdict vector, whatever it holds.

At these sizes the yardstick for the rows is the fp64 evaluation of the reference's formulas
(``measure_row_f64``), not its fp32 CPU evaluation: a plain fp32 sum of 33M squares drifts by
~0.2% (C2's ‖C‖_F: 5782.1 in fp32 against 5792.7 exactly), more than the GPU's error. The
non-negative sums match it to relative 1e-5, honest fp32 residuals within 2 band units, planted
or bf16 residuals to relative 1e-4 with a floor of 2 band units; verdicts are the oracle's
judgement of the fp64 row.
"""

from __future__ import annotations

import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu
FP32, BF16 = 2.0**-24, 2.0**-8


def _verdict(row, q, n, eps_in, biased=False, tau=8.0, kappa=1e4):
    return O.judge(O.finish_row(row, q=q, n=n, eps_in=eps_in, eps_acc=FP32, biased=biased),
                   tau=tau, kappa_max=kappa, guard=True)


def _gpu_verdicts(lib, rows, qs, ns, biased, k, eps_in):
    from verification.commitment import native
    specs = native.verdict_specs(qs, ns, biased, [1e4] * len(qs))
    codes, fin, _ = lib.verdicts(rows, specs, k=k, eps_in=eps_in, eps_acc=FP32, tau=8.0,
                                 finished=True)
    return [tuple(x) for x in codes.cpu().tolist()], fin.cpu().tolist()


@pytest.mark.parametrize("k", [1, 8])
def test_c2_microbench(lib, k):
    from verification.commitment import native
    g = torch.Generator().manual_seed(0)
    # entries N(0, σ² = 1/√4096): C's entries are then N(0, 1)
    a_c = torch.randn(8192, 4096, generator=g) / 8.0
    b_c = torch.randn(4096, 4096, generator=g) / 8.0
    a, b = a_c.cuda(), b_c.cuda()
    c = a @ b
    tampered = c.clone()
    gi = torch.Generator().manual_seed(1)
    i, j = int(torch.randint(0, 8192, (1,), generator=gi)), int(torch.randint(0, 4096, (1,),
                                                                               generator=gi))
    tampered[i, j] *= 1.0 + 1e-2
    for p in (c, tampered):
        p_c = p.cpu()
        want_leaves = [O.tensor_leaf_hash(O.TAG_PRODUCT, t) for t in (a_c, b_c, p_c)]
        root = O.merkle_root(want_leaves)
        # the GPU hashes and roots the three leaves itself
        hdrs = [O.tensor_leaf_header(O.TAG_PRODUCT, t) for t in (a, b, p)]
        plan = lib.leaf_plan(hdrs, [a, b, p], [native.FINITE_KIND[torch.float32]] * 3)
        dig, bad = plan.run()
        got_root = bytes(lib.merkle_tree_device(dig)[0].cpu().numpy())
        assert int(bad.item()) == 3 and got_root == root
        rows = lib.fv_plan([native.FvProduct(a, b, p, 1)], k).rows(root).cpu()[0].tolist()
        r = O.challenge_matrices(root, [1], k, 4096)[0]
        ref64 = O.measure_row_f64(a_c, b_c, p_c, r, None)
        for col in range(5):
            assert rows[col] == pytest.approx(ref64[col], rel=1e-5)
        unit = O.finish_row(ref64, q=4096, n=8192, eps_in=FP32, eps_acc=FP32)["unit"]
        for x, y in zip(rows[5:], ref64[5:]):
            if p is c:
                assert abs(x - y) <= 2 * unit
            else:
                assert x == pytest.approx(y, rel=1e-4, abs=2 * unit)
        codes, _ = _gpu_verdicts(lib, torch.tensor([rows], dtype=torch.float64,
                                                    device="cuda"), [4096], [8192], [False],
                                 k, FP32)
        assert codes[0] == _verdict(ref64, 4096, 8192, FP32)
        assert codes[0][0] == 0  # the honest C, and the tamper below τ, are accepted


def test_c1_full_size(lib):
    from verification.computation.instances import decoder
    from verification.prover.synthetic import synthetic_step
    from verification.verifier.step import DeviceStepVerifier
    c = decoder.smollm2_135m()
    step = synthetic_step(c, seed=0, operands=True)
    items = []
    for i, obj in enumerate(step.leaves):
        if i < c.n_s:
            items.append((b"", torch.frombuffer(bytearray(O.encode_record(
                obj.ids, obj.targets, obj.mask)), dtype=torch.uint8), 0))
        else:
            tag = O.TAG_PRODUCT if c.n_s + c.n_w <= i < c.n_s + c.n_w + c.M else O.TAG_WEIGHT
            t = obj.cpu()
            items.append((O.tensor_leaf_header(tag, t), t, O.FINITE_KIND[t.dtype]))
    hashes, bad = O.hash_leaves(items, 16)
    assert bad == len(items)
    root = O.merkle_root(hashes)
    v = DeviceStepVerifier(c, step.leaves, lambda s: step.operands[s.m], k=1)
    out = v.run(root)
    assert out.root == root and out.check is None, out.detail
    rows = out.rows.cpu().tolist()
    for spec in c.products[::181]:
        a, b = step.operands[spec.m]
        af, bf, pf = a.cpu(), b.cpu(), step.product(spec.m).cpu()
        r = O.challenge_matrices(root, [spec.m], 1, pf.shape[1])[0]
        ref64 = O.measure_row_f64(af, bf, pf, r, None)
        for col in range(5):
            assert rows[spec.m - 1][col] == pytest.approx(ref64[col], rel=1e-5), (spec.name, col)
        unit = O.finish_row(ref64, q=spec.q, n=af.shape[0], eps_in=FP32, eps_acc=FP32)["unit"]
        assert abs(rows[spec.m - 1][5] - ref64[5]) <= 2 * unit, spec.name


def test_c5_adversarial_verdicts(lib):
    from verification.computation.instances.decoder import DecoderComputation
    from verification.prover.synthetic import perturb_products, synthetic_step
    from verification.verifier.step import DeviceStepVerifier
    c = DecoderComputation(L=2, d=1536, d_f=8960, n_h=12, n_kv=2, n_v=4096, n_s=4, n=2048,
                           d_h=128, qkv_bias=True, compute_dtype=torch.bfloat16)
    step = synthetic_step(c, seed=5, operands=True)
    perturbed = {m for m, _, _ in perturb_products(step, 0.05, seed=5)}
    v = DeviceStepVerifier(c, step.leaves, lambda s: step.operands[s.m], k=16)
    root = v.run(bytes(32)).root  # the root a prover committing the forged leaves claims
    out = v.run(root)
    assert out.root == root and out.first_bad == c.n_leaves
    codes = [tuple(x) for x in out.codes.cpu().tolist()]
    rows = out.rows.cpu().tolist()
    checked, borderline, tops = 0, [], {}
    for spec in c.products:
        if spec.m not in perturbed and spec.m % 25:
            continue
        a, b = step.operands[spec.m]
        af, bf, pf = a.float().cpu(), b.float().cpu(), step.product(spec.m).float().cpu()
        bias = None
        if spec.bias is not None:
            bias = step.w_t(spec.bias).to(torch.bfloat16).float().cpu()
        r = O.challenge_matrices(root, [spec.m], 16, pf.shape[1])[0]
        ref64 = O.measure_row_f64(af, bf, pf, r, bias)
        mp = O.finish_row(ref64, q=spec.q, n=af.shape[0], eps_in=BF16, eps_acc=FP32,
                          biased=bias is not None)
        want_code = O.judge(mp, tau=8.0, kappa_max=1e4, guard=True)
        for j in range(16):
            assert rows[spec.m - 1][5 + j] == pytest.approx(ref64[5 + j], rel=1e-4,
                                                            abs=2 * mp["unit"]), (spec.m, j)
        top = tops[spec.m] = max(mp["normalized"])
        if abs(top - 8.0) <= 8e-3:
            borderline.append((spec.m, top, codes[spec.m - 1], want_code))
            continue
        assert codes[spec.m - 1] == want_code, (spec.m, spec.name, top, rows[spec.m - 1])
        checked += 1
    rejected = [m for m in perturbed if codes[m - 1][0] != 0]
    print(f"C5 scaled: {len(perturbed)} perturbed products, {len(rejected)} rejected, "
          f"{checked} verdicts compared, largest perturbed normalized residual "
          f"{max(tops[m] for m in perturbed):.3g}, borderline {borderline}")
    assert checked >= len(perturbed) + c.M // 25 - len(borderline)
    assert all(codes[m - 1][0] == 0 for m in range(1, c.M + 1) if m not in perturbed)
