"""The step transcript as the verifier sees it (reference: verification/transcript/store.py
:67-135 ``TranscriptStore``, :137-240 ``InMemoryStore``; verification/transcript/reader.py
:21-30 ``LeafReader``).

Everything a store serves comes from the prover and is under test: the verifier recomputes
``h`` from :meth:`TranscriptStore.leaf` before trusting :attr:`TranscriptStore.root`, and
takes the leaf count from the declared computation, never from the store.

:class:`InMemoryStore` holds a step's own tensors, which may live in HBM, without copying
them. It records every leaf tensor's ``_version`` when it takes them and raises
:class:`StoreMutationError` on a read of a leaf changed in place since. The on-disk store of
the reference is not part of this build.
"""

from __future__ import annotations

import abc
from collections.abc import Sequence
from typing import Any, Protocol

import torch

from setup.records import Record
from verification.commitment.merkle import MerkleTree
from verification.transcript.errors import StoreMutationError

__all__ = ["LeafReader", "TranscriptStore", "InMemoryStore"]


class LeafReader(Protocol):
    """Read-only access to one step's leaves by 0-based index. The reader reports no leaf
    count: the computation declares it."""

    def leaf(self, index: int) -> Any: ...


def _versions(obj: Any) -> tuple[int, ...]:
    if isinstance(obj, torch.Tensor):
        return (obj._version,)
    if isinstance(obj, Record):
        return (obj.ids._version, obj.targets._version, obj.mask._version)
    return ()


class TranscriptStore(abc.ABC):
    """One step's transcript as the verifier sees it.

    Reading or hashing prover data can raise ``TranscriptFormatError`` and its subclasses,
    ``EncodingError`` and ``NonFiniteError``, a record's ``ValueError`` and ``IndexError``;
    the checks turn each into a rejection at the check that read the leaf.
    """

    @abc.abstractmethod
    def leaf(self, index: int) -> Any:
        """Leaf ``index``: a record object or a tensor."""

    @property
    @abc.abstractmethod
    def root(self) -> bytes:
        """The claimed step commitment ``h``."""

    @abc.abstractmethod
    def path(self, index: int) -> list[bytes]:
        """The claimed audit path of leaf ``index`` into :attr:`root`, nearest sibling first."""

    def dataset_path(self, i: int) -> list[bytes]:
        """The claimed audit path of batch record ``i`` into ``h_D`` (check 4, not part of this
        build)."""
        raise LookupError("this store holds no dataset paths")


class InMemoryStore(TranscriptStore):
    """A committed step's leaves, held by reference (device tensors stay where they are).

    ``root`` defaults to the root of the Merkle tree over the leaves as given in ``tree``;
    ``claimed_root`` overrides it (what a prover claims need not be the tree's root).
    """

    def __init__(self, leaves: Sequence[Any], tree: MerkleTree | None = None,
                 claimed_root: bytes | None = None,
                 dataset_paths: Sequence[Sequence[bytes]] | None = None) -> None:
        if tree is None and claimed_root is None:
            raise ValueError("an in-memory store needs the step's tree or a claimed root")
        self._leaves = list(leaves)
        self._tree = tree
        self._root = claimed_root
        self._versions = [_versions(x) for x in self._leaves]
        self._dataset_paths = (None if dataset_paths is None
                               else tuple(tuple(bytes(h) for h in p) for p in dataset_paths))

    def leaf(self, index: int) -> Any:
        if not 0 <= index < len(self._leaves):
            raise IndexError(f"leaf {index} outside 0..{len(self._leaves) - 1}")
        obj = self._leaves[index]
        if _versions(obj) != self._versions[index]:
            raise StoreMutationError(f"leaf {index} changed in place after the handoff")
        return obj

    @property
    def root(self) -> bytes:
        if self._root is not None:
            return self._root
        assert self._tree is not None
        return self._tree.root

    def path(self, index: int) -> list[bytes]:
        if self._tree is None:
            raise LookupError("this store holds no tree")
        return self._tree.path(index)

    def dataset_path(self, i: int) -> list[bytes]:
        if self._dataset_paths is None:
            raise LookupError("this store holds no dataset paths")
        return list(self._dataset_paths[i])
