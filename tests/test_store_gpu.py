"""A stored step verified from disk, through the reference's store and through the native
loader into HBM (reference tests/verification/transcript/test_store.py:449-474).

A step's leaves written by DiskStore must read back, through DiskStore.leaf (host tensors)
and through load_step (one HBM arena), to the leaves committed, bit for bit; the verifier
must decide a stored step as it decides the step in memory, over either store: accept an
honest step with the same check-5 rows, reject a corrupt leaf file as malformed at check 2,
and a changed product file at check 5. Roots are checked against the CPU oracle.
"""

from __future__ import annotations

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


def _oracle_root(c, leaves):
    want = []
    for i, obj in enumerate(leaves):
        if i < c.n_s:
            want.append(O.hash_leaf(O.encode_record(obj.ids, obj.targets, obj.mask)))
        else:
            tag = O.TAG_PRODUCT if c.n_s + c.n_w <= i < c.n_s + c.n_w + c.M else O.TAG_WEIGHT
            want.append(O.tensor_leaf_hash(tag, obj.cpu()))
    return O.merkle_root(want)


def _stored(tmp_path, seed):
    from verification.commitment.leaves import commit_leaves_device
    from verification.transcript.loader import write_operands
    from verification.transcript.store import DiskStore
    c, step = _step(seed)
    tree = commit_leaves_device(c, step.leaves)
    disk = DiskStore.write(tmp_path / "step", c, step.leaves, tree)
    write_operands(disk.directory, step.operands)
    return c, step, tree, disk


def _same(a, b):
    if isinstance(a, torch.Tensor):
        return (isinstance(b, torch.Tensor) and a.dtype == b.dtype and a.shape == b.shape
                and a.stride() == b.stride() and torch.equal(a.cpu(), b.cpu()))
    return all(torch.equal(getattr(a, k), getattr(b, k)) for k in ("ids", "targets", "mask"))


def test_stored_step_reads_back_bit_for_bit(lib, tmp_path):
    from verification.commitment.merkle import verify_path
    from verification.transcript.loader import load_step
    c, step, tree, disk = _stored(tmp_path, 21)
    assert disk.root == tree.root == _oracle_root(c, step.leaves)
    ms = [s.m for s in c.products]
    res = load_step(disk, c.n_leaves, operand_ms=ms, threads=4, staging_mib=8)
    assert res.fallback == c.n_s  # only the records go through torch.load
    assert res.arena.is_cuda
    for i in range(c.n_leaves):
        assert _same(disk.leaf(i), step.leaves[i])
        assert _same(res.leaves[i], step.leaves[i])
        if isinstance(step.leaves[i], torch.Tensor):
            assert res.leaves[i].is_cuda
    for m in ms:
        for got, want in zip(res.operands[m], step.operands[m]):
            assert got.is_cuda and got.dtype == want.dtype and torch.equal(got, want)
    for i in (0, c.n_s, c.n_leaves - 1):
        assert disk.path(i) == tree.path(i)
        assert verify_path(tree.leaf(i), i, c.n_leaves, disk.path(i), disk.root)


def test_verifier_decides_a_stored_step_as_in_memory(lib, tmp_path):
    from verification.transcript.loader import ResidentStore, load_step
    from verification.transcript.store import InMemoryStore
    from conftest import started_verifier
    c, step, tree, disk = _stored(tmp_path, 22)
    res = load_step(disk, c.n_leaves)
    stats = []
    for store in (InMemoryStore(step.leaves, tree), disk, ResidentStore(disk, res)):
        v = started_verifier(c, step.leaves, k=2)
        assert v.verify_step(1, store) is None
        stats.append([(s.m, s.normalized, s.kappa, s.p_norm, s.p_abs1)
                      for s in v.stats[1].products])
    assert stats[0] == stats[1] == stats[2]


def test_device_step_verifier_on_a_loaded_step(lib, tmp_path):
    from verification.transcript.loader import load_step
    from verification.verifier.step import DeviceStepVerifier
    c, step, tree, disk = _stored(tmp_path, 23)
    res = load_step(disk, c.n_leaves, operand_ms=[s.m for s in c.products])
    dw = DeviceStepVerifier(c, step.leaves, lambda s: step.operands[s.m], k=2)
    dg = DeviceStepVerifier(c, res.leaves, lambda s: res.operands[s.m], k=2)
    want, got = dw.run(tree.root), dg.run(disk.root)
    assert got.check is None and want.check is None, got.detail
    assert got.root == want.root == tree.root
    assert (got.first_bad, got.first_fail) == (c.n_leaves, c.M)
    assert torch.equal(got.codes.cpu(), want.codes.cpu())
    # In memory, a twin's A is a transposed view of its mate's (one read of X measures both);
    # the loaded operands are files of their own, so the loaded plan measures every twin apart.
    # Those rows agree to fp32 rounding (the sums run in another order), the rest bit for bit.
    assert dw.plan.twins > 0 and dg.plan.twins == 0
    index = {s.m: i for i, s in enumerate(c.products)}
    twin = sorted(index[m] for pair in c.operand_twins.items() for m in pair)
    rest = [i for i in range(c.M) if i not in set(twin)]
    gr, wr = got.rows.cpu(), want.rows.cpu()
    assert torch.equal(gr[rest], wr[rest])
    assert torch.allclose(gr[twin, :5], wr[twin, :5], rtol=1e-5, atol=0)
    assert torch.allclose(gr[twin, 5:], wr[twin, 5:], rtol=1e-3, atol=1e-12)


def test_corrupt_leaf_file_rejects_as_malformed(lib, tmp_path):
    from verification.transcript.loader import ResidentStore, load_step
    from verification.transcript.store import LEAF_FILE
    from conftest import started_verifier
    c, step, tree, disk = _stored(tmp_path, 24)
    (disk.directory / LEAF_FILE.format(c.product_index(2))).write_bytes(b"\0" * 10)
    res = load_step(disk, c.n_leaves)
    for store in (disk, ResidentStore(disk, res)):
        rej = started_verifier(c, step.leaves, k=2).verify_step(1, store)
        assert rej is not None and (rej.step, rej.check_id, rej.kind) == (1, "2", "malformed")
        assert "LeafReadError" in rej.detail


def test_changed_product_file_rejects_at_check_5(lib, tmp_path):
    from verification.transcript.loader import ResidentStore, load_step
    from verification.transcript.store import LEAF_FILE
    from conftest import started_verifier
    c, step, tree, disk = _stored(tmp_path, 25)
    spec = c.products[len(c.products) // 3]
    p = step.product(spec.m).clone()
    p[1, 2] += 8.0
    torch.save(p.cpu(), disk.directory / LEAF_FILE.format(c.product_index(spec.m)))
    res = load_step(disk, c.n_leaves)
    details = []
    for store in (disk, ResidentStore(disk, res)):
        rej = started_verifier(c, step.leaves, k=2).verify_step(1, store)
        assert rej is not None and (rej.check_id, rej.kind) == ("5", "failed")
        assert rej.detail.startswith(f"P_{spec.m} ({spec.name})")
        details.append(rej.detail)
    assert details[0] == details[1]
