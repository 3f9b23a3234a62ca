"""TEST INFRASTRUCTURE — a second, independent BLAKE3, in pure Python, for small inputs.

Written from the BLAKE3 specification like ``blake3_spec.c``, but it builds the tree by the
specification's recursive definition instead of a chaining-value stack: a run of ``n > 1``
chunks splits into a left subtree of the largest power of two of chunks below ``n`` and a
right subtree of the rest. The two implementations share nothing but the compression
function, which the reference's known-answer tests pin
(``tests/verification/verifier/matmul_check/test_challenges.py:117-137``,
``tests/verification/commitment/test_merkle.py:27-34``). Agreement between them on
multi-chunk inputs pins the tree.

Slow (pure Python): meant for messages up to a few hundred KiB.
"""

from __future__ import annotations

import struct

IV = (0x6A09E667, 0xBB67AE85, 0x3C6EF372, 0xA54FF53A,
      0x510E527F, 0x9B05688C, 0x1F83D9AB, 0x5BE0CD19)
PERM = (2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8)
CHUNK_START, CHUNK_END, PARENT, ROOT, KEYED_HASH = 1, 2, 4, 8, 16
M32 = 0xFFFFFFFF


def _rotr(x: int, n: int) -> int:
    return ((x >> n) | (x << (32 - n))) & M32


def _g(s: list[int], a: int, b: int, c: int, d: int, mx: int, my: int) -> None:
    s[a] = (s[a] + s[b] + mx) & M32
    s[d] = _rotr(s[d] ^ s[a], 16)
    s[c] = (s[c] + s[d]) & M32
    s[b] = _rotr(s[b] ^ s[c], 12)
    s[a] = (s[a] + s[b] + my) & M32
    s[d] = _rotr(s[d] ^ s[a], 8)
    s[c] = (s[c] + s[d]) & M32
    s[b] = _rotr(s[b] ^ s[c], 7)


def compress(cv: tuple[int, ...], words: tuple[int, ...], counter: int, block_len: int,
             flags: int) -> list[int]:
    """The 16 output words of one compression."""
    s = [*cv, *IV[:4], counter & M32, (counter >> 32) & M32, block_len, flags]
    m = list(words)
    for r in range(7):
        _g(s, 0, 4, 8, 12, m[0], m[1])
        _g(s, 1, 5, 9, 13, m[2], m[3])
        _g(s, 2, 6, 10, 14, m[4], m[5])
        _g(s, 3, 7, 11, 15, m[6], m[7])
        _g(s, 0, 5, 10, 15, m[8], m[9])
        _g(s, 1, 6, 11, 12, m[10], m[11])
        _g(s, 2, 7, 8, 13, m[12], m[13])
        _g(s, 3, 4, 9, 14, m[14], m[15])
        if r < 6:
            m = [m[PERM[i]] for i in range(16)]
    return [s[i] ^ s[i + 8] for i in range(8)] + [s[i + 8] ^ cv[i] for i in range(8)]


def _words(block: bytes) -> tuple[int, ...]:
    return struct.unpack("<16I", block.ljust(64, b"\0"))


class _Node:
    """A node's last compression, not yet run: the chaining value or the root output comes
    from it."""

    __slots__ = ("cv", "words", "counter", "block_len", "flags")

    def __init__(self, cv, words, counter, block_len, flags):
        self.cv, self.words, self.counter = cv, words, counter
        self.block_len, self.flags = block_len, flags

    def chaining_value(self) -> tuple[int, ...]:
        return tuple(compress(self.cv, self.words, self.counter, self.block_len,
                              self.flags)[:8])


def _chunk(data: bytes, index: int, key: tuple[int, ...], flags: int) -> _Node:
    blocks = [data[i:i + 64] for i in range(0, len(data), 64)] or [b""]
    cv = key
    for b, block in enumerate(blocks[:-1]):
        f = flags | (CHUNK_START if b == 0 else 0)
        cv = tuple(compress(cv, _words(block), index, 64, f)[:8])
    last = blocks[-1]
    f = flags | CHUNK_END | (CHUNK_START if len(blocks) == 1 else 0)
    return _Node(cv, _words(last), index, len(last), f)


def _subtree(data: bytes, lo: int, hi: int, key: tuple[int, ...], flags: int) -> _Node:
    """The node over chunks ``[lo, hi)`` of ``data`` by the recursive split."""
    if hi - lo == 1:
        return _chunk(data[1024 * lo:1024 * hi], lo, key, flags)
    k = 1 << ((hi - lo - 1).bit_length() - 1)
    left = _subtree(data, lo, lo + k, key, flags).chaining_value()
    right = _subtree(data, lo + k, hi, key, flags).chaining_value()
    return _Node(key, (*left, *right), 0, 64, flags | PARENT)


def blake3(data: bytes, *, key: bytes | None = None, length: int = 32, seek: int = 0) -> bytes:
    """BLAKE3 of ``data`` (keyed when ``key`` is given), ``length`` output bytes from ``seek``."""
    if key is None:
        kw, flags = IV, 0
    else:
        if len(key) != 32:
            raise ValueError("key must be 32 bytes")
        kw, flags = struct.unpack("<8I", key), KEYED_HASH
    n = max(1, -(-len(data) // 1024))
    root = _subtree(bytes(data), 0, n, kw, flags)
    out = bytearray()
    t = seek // 64
    while len(out) < (seek % 64) + length:
        w = compress(root.cv, root.words, t, root.block_len, root.flags | ROOT)
        out += struct.pack("<16I", *w)
        t += 1
    return bytes(out[seek % 64:seek % 64 + length])
