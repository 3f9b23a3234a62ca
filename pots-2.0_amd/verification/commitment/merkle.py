"""BLAKE3 Merkle tree with RFC 6962 shape (reference: verification/commitment/merkle.py).

``H_leaf(x) = BLAKE3(0x00 ‖ x)``, ``H_node(l, r) = BLAKE3(0x01 ‖ l ‖ r)``. A range of
``n > 1`` leaves splits at the largest power of two strictly below ``n``; an unpaired node is
promoted, not duplicated. Every hash here is computed by the gfx950 kernels of
``libpots_mi355x.so``: leaf messages by the leaf-hashing kernel, nodes by the tree kernel.
The names, arguments, return values and errors are the reference's.
"""

from __future__ import annotations

from collections.abc import Iterable, Sequence

import numpy as np
import torch

from setup.records import Record, encode_record
from verification.commitment import native
from verification.commitment.encoding import tensor_leaf_header, tensor_leaf_payload

DIGEST_SIZE = 32

LeafParts = Sequence[bytes | memoryview]


def _messages_digests(msgs: Sequence[bytes]) -> list[bytes]:
    """``BLAKE3(0x00 ‖ m)`` of each host message, one GPU call for all of them."""
    if not msgs:
        return []
    n = len(msgs)
    lens = np.fromiter((len(m) for m in msgs), dtype=np.uint32, count=n)
    offs = np.zeros(n, dtype=np.uint64)
    if n > 1:
        offs[1:] = np.cumsum(lens[:-1], dtype=np.uint64)
    digests, bad = native.get().hash_leaves(
        b"".join(msgs), offs, lens, np.arange(n, dtype=np.uint32),
        np.zeros(n, dtype=np.uint64), np.zeros(n, dtype=np.uint64),
        np.zeros(n, dtype=np.uint8))
    assert bad == n
    return [bytes(d) for d in digests]


def _joined(parts: Sequence[bytes | memoryview]) -> bytes:
    return b"".join(bytes(memoryview(p)) for p in parts)


def hash_leaf(*parts: bytes | memoryview) -> bytes:
    """BLAKE3(0x00 ‖ parts…)."""
    return _messages_digests([_joined(parts)])[0]


def hash_leaves_until_error(leaves: Iterable[LeafParts]) -> tuple[list[bytes], Exception | None]:
    """``hash_leaf(*parts)`` for each item in order, up to the first error:
    ``(digests of the leaves before it, the error or None)``.

    Items are consumed (and their parts read) on the calling thread in order; an item whose
    parts are not bytes-like is the error at its position, as is an error the iterable raises.
    The items before the first error are hashed in one GPU call.
    """
    msgs: list[bytes] = []
    err: Exception | None = None
    try:
        for item in leaves:
            try:
                msgs.append(_joined(item))
            except Exception as e:
                err = e
                break
    except Exception as e:
        err = e
    return _messages_digests(msgs), err


def hash_leaves(leaves: Iterable[LeafParts]) -> list[bytes]:
    """``hash_leaf(*parts)`` for each item, in order; raises the first error a loop would."""
    digests, err = hash_leaves_until_error(leaves)
    if err is not None:
        raise err
    return digests


def hash_node(left: bytes, right: bytes) -> bytes:
    """BLAKE3(0x01 ‖ left ‖ right): the root of the two-leaf tree over ``left`` and ``right``."""
    return native.get().merkle_tree(bytes(left) + bytes(right), 2)[:DIGEST_SIZE]


def hash_tensor_leaf(tag: int, t: torch.Tensor) -> bytes:
    """Leaf hash of a tensor leaf. A GPU tensor is hashed where it lies."""
    if t.is_cuda:
        from verification.commitment.encoding import (FLOAT_DTYPES, NonFiniteError,
                                                      _check_payload)
        _check_payload(t)
        header = tensor_leaf_header(tag, t)
        digests, bad = native.get().hash_leaves(
            header, np.zeros(1, np.uint64), np.array([len(header)], np.uint32),
            np.zeros(1, np.uint32), np.array([t.data_ptr()], np.uint64),
            np.array([t.nbytes], np.uint64),
            np.array([native.FINITE_KIND[t.dtype]], np.uint8))
        if bad == 0 and t.dtype in FLOAT_DTYPES:
            raise NonFiniteError("float tensor contains NaN or Inf")
        return bytes(digests[0])
    return hash_leaf(tensor_leaf_header(tag, t), tensor_leaf_payload(t))


def hash_record_leaf(rec: Record) -> bytes:
    """Leaf hash of a token record, identical in ``h`` and ``h_D``."""
    return hash_leaf(encode_record(rec))


def _split(n: int) -> int:
    """Largest power of two strictly below ``n`` (n ≥ 2)."""
    return 1 << ((n - 1).bit_length() - 1)


def _check_hashes(leaf_hashes: Sequence[bytes]) -> None:
    if len(leaf_hashes) == 0:
        raise ValueError("a Merkle tree needs at least one leaf")
    for x in leaf_hashes:
        if type(x) is not bytes or len(x) != DIGEST_SIZE:
            raise ValueError("leaf hashes must be 32-byte bytes objects")


def merkle_root(leaf_hashes: Sequence[bytes]) -> bytes:
    """Root over already-hashed leaves (RFC 6962 MTH with BLAKE3)."""
    _check_hashes(leaf_hashes)
    return native.get().merkle_tree(b"".join(leaf_hashes), len(leaf_hashes))[:DIGEST_SIZE]


def merkle_root_device(digests: torch.Tensor) -> torch.Tensor:
    """The root, uint8 ``[32]`` in HBM, of the tree over GPU digests uint8 ``[n, 32]``."""
    return native.get().merkle_tree_device(digests)[0]


def _tree_nodes(leaf_hashes: Sequence[bytes]) -> bytearray:
    """All ``2n − 1`` node hashes in the flat pre-order buffer (node ``p`` at bytes
    ``[32p, 32p + 32)``; a range at ``p`` has its left child at ``p + 1`` and its right child
    at ``p + 2k``, ``k = _split`` of its length)."""
    return bytearray(native.get().merkle_tree(b"".join(leaf_hashes), len(leaf_hashes)))


class MerkleTree:
    """RFC 6962 tree over leaf hashes, caching every subtree hash for O(log n) updates."""

    def __init__(self, leaf_hashes: Sequence[bytes]) -> None:
        _check_hashes(leaf_hashes)
        self._n = len(leaf_hashes)
        self._buf = _tree_nodes(leaf_hashes)

    @classmethod
    def from_nodes(cls, nodes: bytes | bytearray, n: int) -> MerkleTree:
        """A tree from a pre-order node buffer built elsewhere (the GPU tree kernel)."""
        if n < 1 or len(nodes) != DIGEST_SIZE * (2 * n - 1):
            raise ValueError("need 32·(2n − 1) bytes of nodes")
        t = cls.__new__(cls)
        t._n = n
        t._buf = bytearray(nodes)
        return t

    def _at(self, p: int) -> bytes:
        return bytes(self._buf[DIGEST_SIZE * p:DIGEST_SIZE * (p + 1)])

    def _set(self, p: int, h: bytes) -> None:
        self._buf[DIGEST_SIZE * p:DIGEST_SIZE * (p + 1)] = h

    @property
    def root(self) -> bytes:
        return self._at(0)

    @property
    def n_leaves(self) -> int:
        return self._n

    def _index(self, lo: int, hi: int) -> int:
        """Pre-order index of the node for ``[lo, hi)``; ``KeyError`` if there is none."""
        p, nlo, nhi = 0, 0, self._n
        while (nlo, nhi) != (lo, hi):
            if nhi - nlo == 1:
                raise KeyError((lo, hi))
            k = _split(nhi - nlo)
            mid = nlo + k
            if nlo <= lo and hi <= mid:
                p, nhi = p + 1, mid
            elif mid <= lo and hi <= nhi:
                p, nlo = p + 2 * k, mid
            else:
                raise KeyError((lo, hi))
        return p

    def node(self, lo: int, hi: int) -> bytes:
        """Subtree hash of the leaf range ``[lo, hi)``, which must be a node of this tree."""
        return self._at(self._index(lo, hi))

    def leaf(self, i: int) -> bytes:
        self._check_index(i)
        return self._at(self._index(i, i + 1))

    def _check_index(self, i: int) -> None:
        if not 0 <= i < self._n:
            raise IndexError(f"leaf index {i} out of range for {self._n} leaves")

    def _descent(self, i: int) -> tuple[list[tuple[int, int, bool]], int]:
        out = []
        p, lo, hi = 0, 0, self._n
        while hi - lo > 1:
            k = _split(hi - lo)
            left = i < lo + k
            out.append((p, k, left))
            if left:
                p, hi = p + 1, lo + k
            else:
                p, lo = p + 2 * k, lo + k
        return out, p

    def path(self, i: int) -> list[bytes]:
        """RFC 6962 audit path for leaf ``i``, sibling nearest the leaf first."""
        self._check_index(i)
        steps, _ = self._descent(i)
        return [self._at(p + 2 * k if left else p + 1) for p, k, left in reversed(steps)]

    def update_leaf(self, i: int, new_hash: bytes) -> bytes:
        """Replace leaf ``i`` and return the new root, rehashing only its path."""
        self._check_index(i)
        if type(new_hash) is not bytes or len(new_hash) != DIGEST_SIZE:
            raise ValueError("leaf hashes must be 32-byte bytes objects")
        steps, leaf_p = self._descent(i)
        self._set(leaf_p, new_hash)
        for p, k, _ in reversed(steps):
            self._set(p, hash_node(self._at(p + 1), self._at(p + 2 * k)))
        return self.root


def verify_path(leaf_hash: bytes, index: int, n_leaves: int, path: Sequence[bytes],
                root: bytes) -> bool:
    """RFC 9162 §2.1.3.2 inclusion-proof verification with BLAKE3 node hashing."""
    if not 0 <= index < n_leaves:
        return False
    fn, sn, r = index, n_leaves - 1, leaf_hash
    for p in path:
        if sn == 0:
            return False
        if fn & 1 or fn == sn:
            r = hash_node(p, r)
            while not fn & 1 and fn != 0:
                fn >>= 1
                sn >>= 1
        else:
            r = hash_node(r, p)
        fn >>= 1
        sn >>= 1
    return sn == 0 and r == root
