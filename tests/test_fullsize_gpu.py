"""The benchmark's own workloads at full size, against the CPU oracle.

- **C4** (Qwen2-1.5B-shaped step, 4×2048 tokens, bf16 products, k = 4): the transcript the
  bench times, through the same ``DeviceStepVerifier`` with the P pass fused into the leaf
  hasher. Every one of the 9,335 leaf digests and the root must equal the oracle's
  (``native_twin.c`` on the host threads). Rows are compared with the fp64 evaluation of the
  reference's formulas for a sample that holds the head products (Λ [8192,1536]·[1536,151936],
  whose 2.3 GiB leaf has 303,872-byte rows in 1,187 chunk classes; dF; G_E_head), every
  linear product of the first and last layer (the 8960-wide gate/up products and their
  gradients among them) and attention members of every role. The verdict of every product
  must equal the oracle's judgement of its row.
- **C5** (the same transcript, k = 16, a seeded 1% of the products with one entry multiplied
  by 1 ± x, x log-uniform in [1e-6, 1]): the verdict of every perturbed product and of a
  sample of honest ones equal to the oracle's judgement of its fp64 row.
- **C3** (Qwen2-0.5B-shaped step, 8×1024 tokens, bf16, k = 2): digests, root, a row sample
  and every verdict, as for C4.

Tolerances are those of the configuration tests: the non-negative columns relative 1e-5
against fp64; residuals relative 1e-4 with a floor of 2 band units (a bf16 product's own 2⁻⁸
rounding dominates them); digests, roots and verdict codes bit for bit. A product whose
largest normalized residual lies within 0.1% of τ is reported instead of asserted.

Operands are the synthetic capture's (``prover/synthetic.py``), resident in HBM, as in the
bench. The C4 transcript with its operands holds about 151 GiB of HBM.
"""

from __future__ import annotations

import gc
import os
import sys
import time

import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu
FP32, BF16 = 2.0**-24, 2.0**-8
TAU, KAPPA = 8.0, 1e4


def _say(msg: str) -> None:
    print(f"[fullsize] {msg}", file=sys.__stderr__, flush=True)


def _threads() -> int:
    return max(1, min(16, len(os.sched_getaffinity(0))))


def _oracle_digests(c, leaves, batch_bytes: int = 4 << 30) -> list[bytes]:
    """Every leaf's digest by the oracle, leaves copied to the host in batches."""
    out: list[bytes] = []
    items, held = [], 0
    n_prod0, n_prod1 = c.n_s + c.n_w, c.n_s + c.n_w + c.M

    def flush():
        nonlocal items, held
        if items:
            d, bad = O.hash_leaves(items, _threads())
            assert bad == len(items), f"oracle found a non-finite leaf at {len(out) + bad}"
            out.extend(d)
        items, held = [], 0

    for i, obj in enumerate(leaves):
        if i < c.n_s:
            items.append((b"", torch.frombuffer(bytearray(O.encode_record(
                obj.ids, obj.targets, obj.mask)), dtype=torch.uint8), 0))
            continue
        tag = O.TAG_PRODUCT if n_prod0 <= i < n_prod1 else O.TAG_WEIGHT
        t = obj.detach().cpu()
        items.append((O.tensor_leaf_header(tag, t), t, O.FINITE_KIND[t.dtype]))
        held += t.nbytes
        if held >= batch_bytes:
            flush()
    flush()
    return out


def _sample(c, members_per_role: int = 2) -> list:
    """Head products, every linear product of the first and last layer, and the first and
    last members of every attention role in those layers."""
    pick = []
    by_role: dict[tuple[int, str], list] = {}
    for s in c.products:
        if s.layer is None:
            pick.append(s)
        elif s.layer in (1, c.L):
            if s.member is None:
                pick.append(s)
            else:
                by_role.setdefault((s.layer, s.name.split(".")[1].split("[")[0]), []).append(s)
    for specs in by_role.values():
        pick += specs[:members_per_role // 2] + specs[-(members_per_role - members_per_role // 2):]
    return sorted(pick, key=lambda s: s.m)


def _fp64_row(step, spec, root, k):
    a, b = step.operands[spec.m]
    p = step.product(spec.m)
    bias = None
    if spec.bias is not None:  # checks.py:439: the W_t leaf in the operand format
        bias = step.w_t(spec.bias).to(step.c.operand_dtype).float().cpu()
    r = O.challenge_matrices(root, [spec.m], k, p.shape[1], _threads())[0]
    row = O.measure_row_f64(a.cpu(), b.cpu(), p.cpu(), r, bias)
    mp = O.finish_row(row, q=spec.q, n=spec.a_shape[0], eps_in=BF16, eps_acc=FP32,
                      biased=bias is not None)
    return row, mp


def _compare_rows(step, specs, root, k, rows, codes):
    """Rows against the fp64 oracle and verdicts against its judgement; returns the number
    of verdicts compared and the borderline products."""
    compared, borderline = 0, []
    for spec in specs:
        ref, mp = _fp64_row(step, spec, root, k)
        got = rows[spec.m - 1]
        for col in range(5):
            assert got[col] == pytest.approx(ref[col], rel=1e-5, abs=1e-300), \
                (spec.m, spec.name, col, got[col], ref[col])
        for j in range(k):
            assert got[5 + j] == pytest.approx(ref[5 + j], rel=1e-4, abs=2 * mp["unit"]), \
                (spec.m, spec.name, j, got[5 + j], ref[5 + j], mp["unit"])
        want = O.judge(mp, tau=TAU, kappa_max=KAPPA, guard=True)
        top = max(mp["normalized"])
        if abs(top - TAU) <= TAU * 1e-3:
            borderline.append((spec.m, spec.name, top, codes[spec.m - 1], want))
            continue
        assert codes[spec.m - 1] == want, (spec.m, spec.name, top, got)
        compared += 1
    return compared, borderline


def _all_verdicts_match(c, rows, codes):
    """The device verdict of every product equals the oracle's judgement of the device row
    (the closed form of finish_row and _judge_product, fp64)."""
    for spec in c.products:
        row = rows[spec.m - 1]
        mp = O.finish_row(row, q=spec.q, n=spec.a_shape[0], eps_in=BF16, eps_acc=FP32,
                          biased=spec.bias is not None)
        assert codes[spec.m - 1] == O.judge(mp, tau=TAU, kappa_max=KAPPA, guard=True), \
            (spec.m, spec.name, row)


def _free(*objs):
    del objs
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def test_c3_full_size(lib):
    from verification.computation.instances import decoder
    from verification.prover.synthetic import synthetic_step
    from verification.verifier.step import DeviceStepVerifier
    _free()
    c = decoder.qwen2_0_5b_shape()
    step = synthetic_step(c, seed=3, operands=True)
    t0 = time.perf_counter()
    want = _oracle_digests(c, step.leaves)
    root = O.merkle_root(want)
    _say(f"C3 oracle: {len(want)} digests in {time.perf_counter() - t0:.1f} s")
    v = DeviceStepVerifier(c, step.leaves, lambda s: step.operands[s.m], k=2)
    out = v.run(root)
    got = [bytes(x) for x in v.digests.cpu().numpy()]
    bad = [i for i in range(c.n_leaves) if got[i] != want[i]]
    assert not bad, f"{len(bad)} leaf digests differ from the oracle, first {bad[:5]}"
    assert out.root == root and out.check is None, out.detail
    rows = out.rows.cpu().tolist()
    codes = [tuple(x) for x in out.codes.cpu().tolist()]
    _all_verdicts_match(c, rows, codes)
    specs = _sample(c)
    compared, borderline = _compare_rows(step, specs, root, 2, rows, codes)
    _say(f"C3: {compared} rows and verdicts against fp64, borderline {borderline}")
    assert compared >= len(specs) - len(borderline)
    del v, step
    _free()


@pytest.fixture(scope="module")
def c4_step(lib):
    from verification.computation.instances import decoder
    from verification.prover.synthetic import synthetic_step
    c = decoder.qwen2_1_5b_shape()
    t0 = time.perf_counter()
    step = synthetic_step(c, seed=0, operands=True)
    torch.cuda.synchronize()
    _say(f"C4 transcript built in {time.perf_counter() - t0:.1f} s: {c.n_leaves} leaves, "
         f"{c.M} products")
    yield step
    step.leaves.clear()
    step.operands.clear()
    _free()


def test_c4_full_size(lib, c4_step):
    from verification.verifier.step import DeviceStepVerifier
    step, c = c4_step, c4_step.c
    t0 = time.perf_counter()
    want = _oracle_digests(c, step.leaves)
    root = O.merkle_root(want)
    _say(f"C4 oracle: {len(want)} digests in {time.perf_counter() - t0:.1f} s, "
         f"root {root.hex()[:16]}")
    v = DeviceStepVerifier(c, step.leaves, lambda s: step.operands[s.m], k=4)
    assert v.fused, "the bench's configuration fuses the P pass at k = 4"
    hp = v.hasher.plan
    # the 3,223 products with rows of at least 1 KiB (46.8 GB of P) take the fused pass
    assert hp.fused > 3000 and hp.fused_bytes > 45e9, (hp.fused, hp.fused_bytes)
    out = v.run(root)
    got = [bytes(x) for x in v.digests.cpu().numpy()]
    bad = [i for i in range(c.n_leaves) if got[i] != want[i]]
    assert not bad, f"{len(bad)} leaf digests differ from the oracle, first {bad[:5]}"
    assert out.root == root and out.first_bad == c.n_leaves
    assert out.check is None, out.detail
    rows = out.rows.cpu().tolist()
    codes = [tuple(x) for x in out.codes.cpu().tolist()]
    _all_verdicts_match(c, rows, codes)
    specs = _sample(c)
    names = {s.name for s in specs}
    assert {"Lambda", "dF", "G_E_head", "L1.Y_gate", "L1.G_up", "L28.dX_down"} <= names
    t0 = time.perf_counter()
    compared, borderline = _compare_rows(step, specs, root, 4, rows, codes)
    _say(f"C4: {compared} rows and verdicts against fp64 in {time.perf_counter() - t0:.1f} s "
         f"({hp.fused} fused leaves, {hp.fused_bytes / 1e9:.1f} GB), borderline {borderline}")
    assert compared >= len(specs) - len(borderline)
    del v
    _free()


def test_c5_full_size(lib, c4_step):
    """Runs after C4 on the same transcript, which it perturbs in place."""
    from verification.prover.synthetic import perturb_products
    from verification.verifier.step import DeviceStepVerifier
    step, c = c4_step, c4_step.c
    perturbed = {m: (idx, f) for m, idx, f in perturb_products(step, 0.01, seed=5)}
    assert len(perturbed) == round(0.01 * c.M)
    v = DeviceStepVerifier(c, step.leaves, lambda s: step.operands[s.m], k=16)
    root = v.run(bytes(32)).root  # the root a prover committing the forged leaves claims
    out = v.run(root)
    assert out.root == root and out.first_bad == c.n_leaves
    rows = out.rows.cpu().tolist()
    codes = [tuple(x) for x in out.codes.cpu().tolist()]
    _all_verdicts_match(c, rows, codes)
    by_m = {s.m: s for s in c.products}
    specs = sorted({by_m[m] for m in perturbed} | set(_sample(c, 1)), key=lambda s: s.m)
    t0 = time.perf_counter()
    compared, borderline = _compare_rows(step, specs, root, 16, rows, codes)
    rejected = sorted(m for m in perturbed if codes[m - 1][0] != 0)
    _say(f"C5: {len(perturbed)} perturbed, {len(rejected)} rejected; {compared} verdicts "
         f"against fp64 in {time.perf_counter() - t0:.1f} s; borderline {borderline}")
    assert compared >= len(specs) - len(borderline)
    # an honest product is never rejected; the first rejection is the device's first fail
    assert all(codes[m - 1][0] == 0 for m in range(1, c.M + 1) if m not in perturbed)
    assert out.first_fail == (rejected[0] - 1 if rejected else c.M)
    del v
    _free()
