"""Parity of the gfx950 leaf-hashing and Merkle-tree kernels with the CPU oracle: digests,
first-bad indices and roots bit for bit, on the reference's edge shapes and error cases
(tests/verification/commitment/test_native.py, test_merkle.py, test_leaves_native.py)."""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
from payloads import DTYPES, payload  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _tensor_batch(lib, ts, tag=3, device=True):
    """Hash tensors through Native.hash_leaves (the reference's entry point)."""
    from verification.commitment import native
    ts = [t.to(DEV) if device else t for t in ts]
    hdrs = [O.tensor_leaf_header(tag, t) for t in ts]
    hdr_len = np.array([len(h) for h in hdrs], np.uint32)
    hdr_off = np.concatenate([[0], np.cumsum(hdr_len[:-1])]).astype(np.uint64)
    ptr = np.array([t.data_ptr() for t in ts], np.uint64)
    ln = np.array([t.nbytes for t in ts], np.uint64)
    kind = np.array([native.FINITE_KIND[t.dtype] for t in ts], np.uint8)
    d, bad = lib.hash_leaves(b"".join(hdrs), hdr_off, hdr_len, np.arange(len(ts), dtype=np.uint32),
                             ptr, ln, kind)
    return [bytes(x) for x in d], bad


def _expected(ts, tag=3):
    return [O.tensor_leaf_hash(tag, t.cpu()) for t in ts]


def test_golden_digests_single_and_batched(lib):
    from verification.commitment.merkle import hash_tensor_leaf
    entries = json.loads((GOLDEN / "leaf_digests.json").read_text())
    ts = [payload(tuple(e["shape"]), DTYPES[e["dtype"]], e["seed"]) for e in entries]
    for e, t in zip(entries[:40], ts[:40]):
        assert hash_tensor_leaf(e["tag"], t.to(DEV)).hex() == e["digest"], e
    by_tag = {}
    for e, t in zip(entries, ts):
        by_tag.setdefault(e["tag"], []).append((e, t))
    for tag, pairs in by_tag.items():
        got, bad = _tensor_batch(lib, [t for _, t in pairs], tag=tag)
        assert bad == len(pairs)
        assert [g.hex() for g in got] == [e["digest"] for e, _ in pairs]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.int32])
def test_random_shapes_match_oracle(lib, dtype):
    rng = np.random.default_rng(7)
    ts = []
    for i in range(60):
        nd = int(rng.integers(1, 5))
        shape = tuple(int(x) for x in rng.integers(1, 40, nd))
        ts.append(payload(shape, dtype, 500 + i))
    got, bad = _tensor_batch(lib, ts)
    assert bad == len(ts)
    assert got == _expected(ts)


def test_large_leaf_and_prefix(lib):
    for dtype in (torch.float32, torch.bfloat16):
        t = payload(((20 << 20) // dtype.itemsize + 3,), dtype, 3)
        got, bad = _tensor_batch(lib, [t, t[:5].clone()])
        assert bad == 2
        assert got == _expected([t, t[:5]])


def test_views_of_one_storage_and_unaligned_views(lib):
    big = payload((64, 33, 7), torch.float32, 1).to(DEV)
    ts = list(big.unbind(0))
    got, bad = _tensor_batch(lib, ts)
    assert bad == len(ts) and got == _expected(ts)
    # bf16 rows at odd element offsets: 2-byte aligned payloads take the staged path
    flat = payload((4097,), torch.bfloat16, 2).to(DEV)
    views = [flat[i:i + 1000] for i in (0, 1, 2, 3, 5, 7, 1001)]
    got, bad = _tensor_batch(lib, views)
    assert bad == len(views) and got == _expected(views)


def test_tree_shapes_across_fold_boundaries(lib):
    """Leaves of n chunks around the powers of two where the per-leaf tree is reduced several
    levels per launch (2, 3, 8, 9, 64, 65, 512, 513, 4096, 4097 chunks, ...), batched with
    one-chunk leaves between them so that launch blocks span many leaves."""
    counts = [2, 3, 4, 5, 7, 8, 9, 15, 16, 17, 31, 33, 63, 64, 65, 127, 129, 511, 512, 513,
              1023, 1025, 4095, 4096, 4097, 9000]
    ts = []
    for i, n in enumerate(counts):
        # int32 payload of 1024·n − 100 bytes: with its header the message spans n chunks
        ts.append(payload(((1024 * n - 100) // 4,), torch.int32, 900 + i))
        ts.append(payload((3,), torch.float32, 950 + i))
    got, bad = _tensor_batch(lib, ts)
    assert bad == len(ts)
    assert got == _expected(ts)


def test_host_payloads_are_staged(lib):
    ts = [payload((1000 + i,), torch.float32, 40 + i) for i in range(5)]
    got, bad = _tensor_batch(lib, ts, device=False)
    assert bad == len(ts) and got == _expected(ts)


def test_staged_headers_are_not_tested_for_nan(lib):
    """A staged leaf (host payload, or a view not 4-byte aligned) carries its 0x00 || header
    bytes in the staged message; only the payload is NaN/Inf-tested, as in native.c. The
    big-endian dims below put an all-ones exponent into a header half-word or word: 124 for
    fp16 (bytes 00 7C), 32895 = 0x807F for bf16 and fp32."""
    ts = [payload((124,), torch.float16, 1), payload((3, 124), torch.float16, 2),
          payload((32895,), torch.bfloat16, 3), payload((2, 32895), torch.float32, 4),
          payload((32895,), torch.float16, 5)]
    got, bad = _tensor_batch(lib, ts, device=False)
    assert bad == len(ts) and got == _expected(ts)
    for dt, n in ((torch.float16, 124), (torch.bfloat16, 32895), (torch.float16, 32895)):
        flat = payload((n + 1,), dt, 6).to(DEV)
        v = flat[1:]  # 2-byte aligned: staged
        got, bad = _tensor_batch(lib, [v])
        assert bad == 1 and got == _expected([v])
    # the payload of a staged leaf is still tested
    t = payload((124,), torch.float16, 7)
    t[100] = float("inf")
    _, bad = _tensor_batch(lib, [payload((5,), torch.float32, 8), t], device=False)
    assert bad == 1


def test_many_small_leaves(lib):
    ts = [payload((13,), torch.float32, i) for i in range(5000)]
    got, bad = _tensor_batch(lib, ts)
    assert bad == len(ts) and got == _expected(ts)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_first_bad_is_the_first_in_order(lib, dtype):
    rng = np.random.default_rng(5)
    for trial in range(6):
        ts = [payload((300 + 97 * i,), dtype, 60 + i) for i in range(20)]
        for i in (9, 5):
            ts[i] = ts[i].clone()
            ts[i][int(rng.integers(ts[i].numel()))] = [float("nan"), float("inf"),
                                                       -float("inf")][trial % 3]
        got, bad = _tensor_batch(lib, ts)
        assert bad == 5
        assert got[:5] == _expected(ts[:5])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_every_position_of_a_word_is_tested(lib, dtype):
    from verification.commitment import native
    for pos in range(9):
        t = torch.ones(9, dtype=dtype)
        t[pos] = float("inf")
        _, bad = _tensor_batch(lib, [t])
        assert bad == 0
        assert not lib.all_finite(t.to(DEV).data_ptr(), t.nbytes, native.FINITE_KIND[dtype])
    assert lib.all_finite(torch.full((9,), -0.0, dtype=dtype).to(DEV).data_ptr(), 18,
                          native.FINITE_KIND[dtype])


def test_int32_is_never_tested(lib):
    t = torch.full((100,), 0x7F800000, dtype=torch.int32)
    got, bad = _tensor_batch(lib, [t])
    assert bad == 1 and got == _expected([t])


def test_header_only_messages_and_records(lib):
    from verification.commitment.merkle import hash_leaf, hash_leaves, hash_record_leaf
    from setup.records import Record
    for msg in (b"", b"a", b"abc", bytes(range(200)), bytes(5000)):
        assert hash_leaf(msg) == O.hash_leaf(msg)
    parts = [(b"x" * i, memoryview(b"y" * (3 * i))) for i in range(30)]
    assert hash_leaves(parts) == [O.hash_leaf(a + bytes(b)) for a, b in parts]
    ids = torch.arange(257, dtype=torch.int32)
    rec = Record(ids, ids + 1, torch.ones(257, dtype=torch.int32))
    assert hash_record_leaf(rec) == O.hash_leaf(O.encode_record(ids, ids + 1, rec.mask))


def test_hash_leaves_until_error_order(lib):
    from verification.commitment.merkle import hash_leaves_until_error

    def items():
        yield (b"a",)
        yield (b"b",)
        yield (object(),)  # not bytes-like: the error sits at this leaf
        yield (b"c",)
    digests, err = hash_leaves_until_error(items())
    assert digests == [O.hash_leaf(b"a"), O.hash_leaf(b"b")] and isinstance(err, TypeError)


@pytest.mark.parametrize("n", [*range(1, 71), 127, 128, 129, 1000, 4097])
def test_merkle_tree_matches_oracle(lib, n):
    hs = [O.hash_leaf(i.to_bytes(4, "big")) for i in range(n)]
    want = O.merkle_tree(hs)
    assert lib.merkle_tree(b"".join(hs), n) == want
    d = torch.frombuffer(bytearray(b"".join(hs)), dtype=torch.uint8).view(n, 32).to(DEV)
    assert bytes(lib.merkle_tree_device(d).cpu().numpy().tobytes()) == want


def test_merkle_api_matches_oracle(lib):
    from verification.commitment.merkle import (MerkleTree, hash_node, merkle_root,
                                                verify_path)
    hs = [O.hash_leaf(i.to_bytes(4, "big")) for i in range(37)]
    assert hash_node(hs[0], hs[1]) == O.hash_node(hs[0], hs[1])
    assert merkle_root(hs) == O.merkle_root(hs)
    t = MerkleTree(hs)
    for i in range(37):
        assert verify_path(hs[i], i, 37, t.path(i), t.root)
        assert O.verify_path(hs[i], i, 37, t.path(i), t.root)
    new = O.hash_leaf(b"tampered")
    root = t.update_leaf(11, new)
    assert root == O.merkle_root(hs[:11] + [new] + hs[12:])
    with pytest.raises(ValueError):
        merkle_root([hs[0], hs[1][:31]])
    with pytest.raises(ValueError):
        MerkleTree([])


def test_abc_known_answer_on_gpu(lib):
    from verification.commitment.merkle import hash_leaf, merkle_root
    ka = json.loads((GOLDEN / "blake3_known_answers.json").read_text())["reference"]
    hs = [hash_leaf(x.encode()) for x in ka["merkle_abc"]["leaves_ascii"]]
    assert merkle_root(hs).hex() == ka["merkle_abc"]["root"]
