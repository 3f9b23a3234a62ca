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
import os
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


# ---- on disk (the reference's files, store.py:244-380) -----------------------------------

LEAF_FILE = "leaf_{:05d}.pt"
META_FILE = "meta.json"
HASHES_FILE = "leaf_hashes.bin"
DISK_FORMAT = 1
RECORD_KEYS = ("ids", "mask", "targets")  # the dict a record leaf is saved as, keys sorted


def savable(t: torch.Tensor) -> torch.Tensor:
    """A detached tensor that ``torch.save`` writes without foreign bytes: ``torch.save``
    writes a tensor's whole storage, so a view (an attention member of a batched output, a
    record sliced out of ``D``) is copied into a storage of its own first."""
    t = t.detach()
    if t.storage_offset() != 0 or t.untyped_storage().nbytes() != t.nbytes:
        return t.clone()
    return t


def disk_object(obj: Any) -> Any:
    """The object one leaf file holds: the tensor itself, or a record's three tensors as a
    dict keyed by :data:`RECORD_KEYS`."""
    if isinstance(obj, Record):
        return {"ids": savable(obj.ids), "mask": savable(obj.mask),
                "targets": savable(obj.targets)}
    if isinstance(obj, torch.Tensor):
        return savable(obj)
    raise TypeError(f"unsupported leaf object {type(obj).__name__}")


def leaf_object(index: int, obj: Any) -> Any:
    """The leaf a loaded file holds. A tensor is served as it is; a dict with exactly the
    record keys becomes a :class:`Record` (whose own checks raise ``RecordError``); anything
    else is :class:`LeafReadError`."""
    if isinstance(obj, torch.Tensor):
        return obj
    if isinstance(obj, dict) and set(obj) == set(RECORD_KEYS):
        return Record(ids=obj["ids"], targets=obj["targets"], mask=obj["mask"])
    raise LeafReadError(f"leaf {index} holds a {type(obj).__name__}, which is not a leaf")


def _hexes(value: Any, what: str) -> list[bytes]:
    """A JSON list of hex strings as digests' bytes; anything else is :class:`LeafReadError`."""
    if not isinstance(value, list):
        raise LeafReadError(f"{what}: expected a list of hex digests, got "
                            f"{type(value).__name__}")
    out = []
    for x in value:
        if not isinstance(x, str):
            raise LeafReadError(f"{what}: a {type(x).__name__} where a hex digest belongs")
        try:
            out.append(bytes.fromhex(x))
        except ValueError as e:
            raise LeafReadError(f"{what}: {x[:20]!r} is not hex") from e
    return out


class DiskStore(TranscriptStore):
    """One committed step in its own directory, read back file by file.

    :meth:`write` stores a step and opens it; ``DiskStore(directory)`` opens a stored one
    without reading anything. Every :meth:`leaf`, :attr:`root` and path reads its file again,
    so a file that is missing (``IndexError`` for a leaf) or unreadable (:class:`LeafReadError`)
    is prover data that fails at the check reading it. Leaves load with ``weights_only=True``,
    which rebuilds tensors and plain containers and runs nothing else.
    """

    def __init__(self, directory: str | Path) -> None:
        self.directory = Path(directory)

    @classmethod
    def write(cls, directory: str | Path, c: Any, leaves: Sequence[Any], tree: MerkleTree,
              dataset_paths: Sequence[Sequence[bytes]] | None = None) -> DiskStore:
        """Store the committed ``leaves``, their ``tree`` and each record's path into ``h_D``
        as ``directory``, replacing what it held, and open it. The files go into a sibling
        staging directory, the metadata last, which is renamed to ``directory`` only when
        complete: ``directory`` never holds a partial step, and after a failed write it does
        not exist."""
        if dataset_paths is not None and len(dataset_paths) != c.n_s:
            raise ValueError(f"{len(dataset_paths)} dataset paths for {c.n_s} records")
        if len(leaves) != tree.n_leaves:
            raise ValueError(f"{len(leaves)} leaves for a tree of {tree.n_leaves}")
        target = Path(directory)
        staging = target.with_name(f".{target.name}.partial-{os.getpid()}")
        for old in (target, staging):
            if old.exists():
                shutil.rmtree(old)
        staging.mkdir(parents=True)
        try:
            for i, obj in enumerate(leaves):
                torch.save(disk_object(obj), staging / LEAF_FILE.format(i))
            with open(staging / HASHES_FILE, "wb") as f:
                for i in range(tree.n_leaves):
                    f.write(tree.leaf(i))
            meta = {"format": DISK_FORMAT, "root": tree.root.hex(), "dataset_paths": None}
            if dataset_paths is not None:
                meta["dataset_paths"] = [[bytes(h).hex() for h in p] for p in dataset_paths]
            (staging / META_FILE).write_text(json.dumps(meta))
            staging.rename(target)
        except BaseException:
            shutil.rmtree(staging, ignore_errors=True)
            raise
        return cls(target)

    def leaf_path(self, index: int) -> Path:
        return self.directory / LEAF_FILE.format(index)

    def _meta(self) -> dict[str, Any]:
        try:
            meta = json.loads((self.directory / META_FILE).read_text())
        except (OSError, ValueError) as e:
            raise LeafReadError(f"cannot read {META_FILE}: {type(e).__name__}: {e}") from e
        if not isinstance(meta, dict) or meta.get("format") != DISK_FORMAT:
            raise LeafReadError(f"{META_FILE} is not in store format {DISK_FORMAT}")
        return meta

    def leaf(self, index: int) -> Any:
        path = self.leaf_path(index) if isinstance(index, int) and index >= 0 else None
        if path is None or not path.is_file():
            raise IndexError(f"no leaf {index!r} in {self.directory.name}")
        try:
            obj = torch.load(path, map_location="cpu", weights_only=True)
        except Exception as e:  # a file that does not load is bad prover data
            raise LeafReadError(f"leaf {index}: {path.name} does not load "
                                f"({type(e).__name__}: {e})") from e
        return leaf_object(index, obj)

    @property
    def root(self) -> bytes:
        return _hexes([self._meta().get("root")], "the root")[0]

    def leaf_hashes(self) -> list[bytes]:
        """The stored leaf hashes (what the prover claims; the verifier rehashes leaves)."""
        try:
            raw = (self.directory / HASHES_FILE).read_bytes()
        except OSError as e:
            raise LeafReadError(f"cannot read {HASHES_FILE}: {e}") from e
        n, rest = divmod(len(raw), DIGEST_SIZE)
        if n == 0 or rest:
            raise LeafReadError(f"{HASHES_FILE} holds {len(raw)} bytes, not whole digests")
        return [raw[DIGEST_SIZE * i:DIGEST_SIZE * (i + 1)] for i in range(n)]

    def path(self, index: int) -> list[bytes]:
        hashes = self.leaf_hashes()
        if not (isinstance(index, int) and 0 <= index < len(hashes)):
            raise IndexError(f"no leaf {index!r} among {len(hashes)}")
        return MerkleTree(hashes).path(index)

    def dataset_path(self, i: int) -> list[bytes]:
        paths = self._meta().get("dataset_paths")
        if paths is None:
            raise LookupError("this store was written without dataset paths")
        if not isinstance(paths, list):
            raise LeafReadError("the dataset paths are not a list")
        return _hexes(paths[i], f"dataset path {i}")

    def remove(self) -> None:
        """Delete the step's directory."""
        shutil.rmtree(self.directory, ignore_errors=True)


# ---- hand-offs (reference store.py:383-423) -----------------------------------------------


class StoreHandoff(abc.ABC):
    """How a run loop passes step ``t``'s committed leaves to the verifier, and drops the store
    once the step is verified."""

    @abc.abstractmethod
    def hold(self, c: Any, t: int, leaves: list[Any], tree: MerkleTree,
             dataset_paths: Sequence[Sequence[bytes]] | None = None) -> TranscriptStore:
        """The store over the committed ``leaves``."""

    def release(self, store: TranscriptStore) -> None:
        """Drop ``store``. A hand-off that keeps nothing of its own has nothing to do."""
        return None


class InMemoryHandoff(StoreHandoff):
    """The leaves stay where they are; the store keeps references (:meth:`InMemoryStore.hold`)."""

    def hold(self, c: Any, t: int, leaves: list[Any], tree: MerkleTree,
             dataset_paths: Sequence[Sequence[bytes]] | None = None) -> InMemoryStore:
        return InMemoryStore.hold(c, leaves, tree, dataset_paths)


IN_MEMORY = InMemoryHandoff()


class DiskHandoff(StoreHandoff):
    """Each step is written to ``directory/step_<t>/`` and served as a :class:`DiskStore`;
    releasing it deletes that directory unless ``keep``, so a run holds one step on disk."""

    def __init__(self, directory: str | Path, *, keep: bool = False) -> None:
        self.directory, self.keep = Path(directory), keep

    def step_directory(self, t: int) -> Path:
        return self.directory / f"step_{t}"

    def hold(self, c: Any, t: int, leaves: list[Any], tree: MerkleTree,
             dataset_paths: Sequence[Sequence[bytes]] | None = None) -> DiskStore:
        return DiskStore.write(self.step_directory(t), c, leaves, tree, dataset_paths)

    def release(self, store: TranscriptStore) -> None:
        if isinstance(store, DiskStore) and not self.keep:
            store.remove()
