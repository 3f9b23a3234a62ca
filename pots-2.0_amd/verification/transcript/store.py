"""The step transcript as the verifier sees it (reference: verification/transcript/store.py
:67-135 ``TranscriptStore``, :137-240 ``InMemoryStore``; verification/transcript/reader.py
:21-30 ``LeafReader``).

Everything a store serves comes from the prover and is under test: the verifier recomputes
``h`` from :meth:`TranscriptStore.leaf` before trusting :attr:`TranscriptStore.root`, and
takes the leaf count from the declared computation, never from the store.

:class:`InMemoryStore` holds a step's own tensors, which may live in HBM, without copying
them. It records every leaf tensor's ``_version`` when it takes them and raises
:class:`StoreMutationError` on a read of a leaf changed in place since.

:class:`DiskStore` (reference store.py:244-380) serves a step from a directory in the
reference's format, file for file: ``leaf_{i:05d}.pt`` holds leaf ``i`` as ``torch.save``
wrote it (a tensor, or a record as the dict ``{"ids", "mask", "targets"}``); ``meta.json``
holds ``{"format": 1, "root": hex, "dataset_paths": null | [[hex, ...], ...]}``;
``leaf_hashes.bin`` holds the tree's leaf hashes end to end. Every :meth:`DiskStore.leaf`
reads its file again with ``torch.load(weights_only=True)`` into fresh host tensors, so a
missing or corrupt file is prover data that fails at the check reading it. To bring a whole
stored step into HBM at once, :func:`verification.transcript.loader.load_step` reads the
same files natively through pinned staging.

The hand-offs (reference store.py:383-423) are how a run loop turns a committed step into the
store it gives the verifier and discards it afterwards: :data:`IN_MEMORY` keeps references,
:class:`DiskHandoff` writes ``directory/step_<t>/`` and deletes it on release unless
``keep``.
"""

from __future__ import annotations

import abc
import json
import shutil
from collections.abc import Sequence
from pathlib import Path
from typing import Any, Protocol

import torch

from setup.records import Record
from verification.commitment.merkle import DIGEST_SIZE, MerkleTree
from verification.transcript.errors import LeafReadError, StoreMutationError

__all__ = ["LeafReader", "TranscriptStore", "InMemoryStore", "DiskStore", "StoreHandoff",
           "InMemoryHandoff", "IN_MEMORY", "DiskHandoff", "LEAF_FILE", "META_FILE",
           "HASHES_FILE", "DISK_FORMAT"]


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

    @classmethod
    def hold(cls, c: Any, leaves: Sequence[Any], tree: MerkleTree,
             dataset_paths: Sequence[Sequence[bytes]] | None = None) -> InMemoryStore:
        """The store over the leaves a commit produced and their ``tree`` (reference
        store.py:206-213): one dataset path per record of ``c``, if any."""
        if dataset_paths is not None and len(dataset_paths) != c.n_s:
            raise ValueError(f"{len(dataset_paths)} dataset paths for {c.n_s} records")
        return cls(leaves, tree, dataset_paths=dataset_paths)

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


# ---- on disk (reference store.py:244-380) -------------------------------------------------

LEAF_FILE = "leaf_{:05d}.pt"
META_FILE = "meta.json"
HASHES_FILE = "leaf_hashes.bin"
DISK_FORMAT = 1
RECORD_KEYS = ("ids", "mask", "targets")  # the dict a record leaf is saved as, keys sorted


def savable(t: torch.Tensor) -> torch.Tensor:
    """``t`` detached, copied if it does not own exactly its storage: ``torch.save`` writes a
    tensor's whole storage, so a view would carry its base's bytes into the file."""
    t = t.detach()
    owns = t.storage_offset() == 0 and \
        t.untyped_storage().nbytes() == t.numel() * t.element_size()
    return t if owns else t.clone()


def disk_object(obj: Any) -> Any:
    """What ``torch.save`` writes for one leaf: the tensor, or a record's three tensors."""
    if isinstance(obj, torch.Tensor):
        return savable(obj)
    if isinstance(obj, Record):
        return {k: savable(getattr(obj, k)) for k in RECORD_KEYS}
    raise TypeError(f"unsupported leaf object {type(obj).__name__}")


def leaf_object(index: int, obj: Any) -> Any:
    """The leaf a loaded file holds; anything but a tensor or a record's dict is
    :class:`LeafReadError`, and a dict that is no valid record raises ``RecordError``."""
    if isinstance(obj, torch.Tensor):
        return obj
    if isinstance(obj, dict) and tuple(sorted(obj)) == RECORD_KEYS:
        return Record(**obj)
    raise LeafReadError(f"leaf {index}: the stored object is a {type(obj).__name__}, not a leaf")


def _hex_digests(value: Any, what: str) -> list[bytes]:
    if not isinstance(value, list):
        raise LeafReadError(f"{what} is not a list")
    try:
        return [bytes.fromhex(x) for x in value]
    except (TypeError, ValueError) as e:
        raise LeafReadError(f"{what} is not a list of hex digests") from e


class DiskStore(TranscriptStore):
    """One committed step in its directory, read back file by file.

    :meth:`write` stores a step and opens it; ``DiskStore(directory)`` opens a written one and
    reads nothing yet. :meth:`leaf`, :attr:`root` and the paths read their files on every
    call: a file that is missing (``IndexError`` for a leaf) or cannot be read
    (:class:`LeafReadError`) is bad prover data at the check that reads it. Leaves load with
    ``weights_only=True``, which rebuilds tensors and plain containers and runs nothing else.
    """

    def __init__(self, directory: str | Path) -> None:
        self.directory = Path(directory)

    @classmethod
    def write(cls, directory: str | Path, c: Any, leaves: Sequence[Any], tree: MerkleTree,
              dataset_paths: Sequence[Sequence[bytes]] | None = None) -> DiskStore:
        """Store ``leaves`` and their ``tree`` (and each record's path into ``h_D``) in
        ``directory``, replacing what it held. ``meta.json`` goes last, so a directory without
        it is an unfinished write; a write that fails removes the directory."""
        if dataset_paths is not None and len(dataset_paths) != c.n_s:
            raise ValueError(f"{len(dataset_paths)} dataset paths for {c.n_s} records")
        if len(leaves) != tree.n_leaves:
            raise ValueError(f"{len(leaves)} leaves for a tree of {tree.n_leaves}")
        d = Path(directory)
        if d.exists():
            shutil.rmtree(d)
        d.mkdir(parents=True)
        try:
            for i, obj in enumerate(leaves):
                torch.save(disk_object(obj), d / LEAF_FILE.format(i))
            (d / HASHES_FILE).write_bytes(b"".join(tree.leaf(i) for i in range(tree.n_leaves)))
            paths = None if dataset_paths is None else \
                [[bytes(h).hex() for h in p] for p in dataset_paths]
            (d / META_FILE).write_text(json.dumps(
                {"format": DISK_FORMAT, "root": tree.root.hex(), "dataset_paths": paths}))
        except BaseException:
            shutil.rmtree(d, ignore_errors=True)
            raise
        return cls(d)

    def leaf_path(self, index: int) -> Path:
        return self.directory / LEAF_FILE.format(index)

    def _meta(self) -> dict[str, Any]:
        try:
            meta = json.loads((self.directory / META_FILE).read_text())
        except (OSError, ValueError) as e:
            raise LeafReadError(f"store metadata unreadable: {type(e).__name__}: {e}") from e
        if not isinstance(meta, dict) or meta.get("format") != DISK_FORMAT:
            raise LeafReadError("store metadata has an unknown format")
        return meta

    def leaf(self, index: int) -> Any:
        if not isinstance(index, int) or index < 0:
            raise IndexError(f"leaf index {index!r} out of range")
        path = self.leaf_path(index)
        if not path.is_file():
            raise IndexError(f"leaf index {index} out of range (no file {path.name})")
        try:
            obj = torch.load(path, map_location="cpu", weights_only=True)
        except Exception as e:  # an unloadable file is bad prover data, not a verifier bug
            raise LeafReadError(f"leaf {index} unreadable: {type(e).__name__}: {e}") from e
        return leaf_object(index, obj)

    @property
    def root(self) -> bytes:
        return _hex_digests([self._meta().get("root")], "the root")[0]

    def leaf_hashes(self) -> list[bytes]:
        """The stored leaf hashes (what the prover claims; the verifier rehashes leaves)."""
        try:
            raw = (self.directory / HASHES_FILE).read_bytes()
        except OSError as e:
            raise LeafReadError(f"leaf hashes unreadable: {e}") from e
        if not raw or len(raw) % DIGEST_SIZE:
            raise LeafReadError(f"a leaf-hash file of {len(raw)} bytes")
        return [raw[i:i + DIGEST_SIZE] for i in range(0, len(raw), DIGEST_SIZE)]

    def path(self, index: int) -> list[bytes]:
        hashes = self.leaf_hashes()
        if not 0 <= index < len(hashes):
            raise IndexError(f"leaf index {index} out of range")
        return MerkleTree(hashes).path(index)

    def dataset_path(self, i: int) -> list[bytes]:
        paths = self._meta().get("dataset_paths")
        if paths is None:
            raise LookupError("this store was written without dataset paths")
        if not isinstance(paths, list):
            raise LeafReadError("the dataset paths are not a list")
        return _hex_digests(paths[i], f"dataset path {i}")

    def remove(self) -> None:
        """Delete the step's directory."""
        shutil.rmtree(self.directory, ignore_errors=True)


# ---- hand-offs (reference store.py:383-423) -----------------------------------------------


class StoreHandoff(abc.ABC):
    """How a run loop gives step ``t``'s committed leaves to the verifier, and discards the
    store once the step is verified."""

    @abc.abstractmethod
    def hold(self, c: Any, t: int, leaves: list[Any], tree: MerkleTree,
             dataset_paths: Sequence[Sequence[bytes]] | None = None) -> TranscriptStore:
        """The store over the committed ``leaves``."""

    def release(self, store: TranscriptStore) -> None:  # noqa: B027 (nothing to free in memory)
        """Discard ``store``."""


class InMemoryHandoff(StoreHandoff):
    """Keep references to the leaves (:meth:`InMemoryStore.hold`)."""

    def hold(self, c: Any, t: int, leaves: list[Any], tree: MerkleTree,
             dataset_paths: Sequence[Sequence[bytes]] | None = None) -> InMemoryStore:
        return InMemoryStore.hold(c, leaves, tree, dataset_paths)


IN_MEMORY = InMemoryHandoff()


class DiskHandoff(StoreHandoff):
    """Write each step to ``directory/step_<t>/`` and serve it as a :class:`DiskStore`;
    :meth:`release` deletes the step's directory unless ``keep``."""

    def __init__(self, directory: str | Path, *, keep: bool = False) -> None:
        self.directory = Path(directory)
        self.keep = keep

    def hold(self, c: Any, t: int, leaves: list[Any], tree: MerkleTree,
             dataset_paths: Sequence[Sequence[bytes]] | None = None) -> DiskStore:
        return DiskStore.write(self.directory / f"step_{t}", c, leaves, tree, dataset_paths)

    def release(self, store: TranscriptStore) -> None:
        if not self.keep and isinstance(store, DiskStore):
            store.remove()
