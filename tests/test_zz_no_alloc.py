"""The allocation-free entry point ``pots_hash_leaves_noalloc`` against ``pots_hash_leaves``,
through the C ABI: the same digests and first-bad index bit for bit, on two calls in a row
(the second smaller, so it runs over the first call's leftovers in the shared scratch), for
device and host payloads, a NaN leaf, and a request larger than the scratch, which is
refused before any GPU work."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu
SIZE_MAX = (1 << 64) - 1


def _call(lib, name, leaves, kinds):
    """Call ``name`` through ctypes with every leaf a product leaf (tag 0x03)."""
    hdrs = [O.tensor_leaf_header(O.TAG_PRODUCT, t) for t in leaves]
    hb = np.frombuffer(b"".join(hdrs), dtype=np.uint8)
    hlen = np.array([len(h) for h in hdrs], dtype=np.uint32)
    hoff = np.concatenate([[0], np.cumsum(hlen[:-1])]).astype(np.uint64)
    hidx = np.arange(len(leaves), dtype=np.uint32)
    ptr = np.array([t.data_ptr() for t in leaves], dtype=np.uint64)
    ln = np.array([t.nbytes for t in leaves], dtype=np.uint64)
    kd = np.array(kinds, dtype=np.uint8)
    out = np.zeros((len(leaves), 32), dtype=np.uint8)
    fn = getattr(lib._lib, name)
    addr = [a.ctypes.data for a in (hb, hoff, hlen, hidx, ptr, ln, kd, out)]
    bad = fn(len(leaves), *map(ctypes.c_void_p, addr), 1)
    return out, bad


def _leaves(seed, sizes, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    out = []
    for i, n in enumerate(sizes):
        dt = (torch.float32, torch.bfloat16)[i % 2]
        out.append(torch.randn(n, generator=g).to(dt).to(device).reshape(-1, 1)
                   if n % 2 else torch.randn(n // 2, 2, generator=g).to(dt).to(device))
    return out


def _kinds(leaves):
    return [{torch.float32: 1, torch.bfloat16: 2}[t.dtype] for t in leaves]


def test_noalloc_equals_the_allocating_entry_point(lib):
    big = _leaves(1, [1, 255, 256, 257, 1 << 16, (1 << 20) + 3, 3 << 20, 517, 4096])
    small = _leaves(2, [7, 300, 1 << 12])
    for leaves in (big, small):  # the second call is smaller
        want, want_bad = _call(lib, "pots_hash_leaves", leaves, _kinds(leaves))
        got, got_bad = _call(lib, "pots_hash_leaves_noalloc", leaves, _kinds(leaves))
        assert got_bad == want_bad == len(leaves)
        assert np.array_equal(got, want)
        assert [bytes(x) for x in got] == [O.tensor_leaf_hash(O.TAG_PRODUCT, t.cpu())
                                           for t in leaves]


def test_noalloc_host_payloads_and_first_bad(lib):
    leaves = _leaves(3, [100, 5000, 70000, 33], device="cpu")
    leaves[2].view(-1)[123] = float("nan")
    want, want_bad = _call(lib, "pots_hash_leaves", leaves, _kinds(leaves))
    got, got_bad = _call(lib, "pots_hash_leaves_noalloc", leaves, _kinds(leaves))
    assert got_bad == want_bad == 2
    assert np.array_equal(got[:2], want[:2])


def test_noalloc_refuses_more_than_its_scratch(lib):
    huge = torch.zeros(3 << 30, dtype=torch.uint8, device="cuda").view(torch.float32)
    _, bad = _call(lib, "pots_hash_leaves_noalloc", [huge.view(-1, 1024)], [1])
    assert bad == SIZE_MAX
    assert "bytes of device scratch" in lib._lib.pots_last_error().decode()
    del huge
    torch.cuda.empty_cache()
    # the entry point still works after the refusal
    leaves = _leaves(4, [999, 12345])
    want, _ = _call(lib, "pots_hash_leaves", leaves, _kinds(leaves))
    got, bad = _call(lib, "pots_hash_leaves_noalloc", leaves, _kinds(leaves))
    assert bad == 2 and np.array_equal(got, want)
