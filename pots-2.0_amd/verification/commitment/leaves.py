"""Leaf encoding and hashing for the step root ``h`` and the dataset root ``h_D``.

Reference: verification/commitment/leaves.py. A leaf is encoded by its position in the
computation's layout: records through ``c.encode_record``, weights with tag 0x02, products
with tag 0x03. Bulk hashing validates each leaf's slot (shape, dtype) on the calling thread,
in order, and hashes the leaves in one GPU call per batch; the digests and the first error are
those of a leaf-by-leaf loop: a structural error stops the walk at its leaf, and the first
leaf whose payload holds NaN or Inf raises ``NonFiniteError`` after the digests before it.

Leaves may be CPU or GPU tensors. GPU payloads are hashed in place in HBM; CPU payloads are
copied to the GPU by the library as part of the call. :func:`hash_step_leaves_device` and
:func:`commit_leaves_device` keep a resident transcript and its digests on the GPU.
"""

from __future__ import annotations

import weakref
from collections.abc import Iterable, Sequence
from time import perf_counter
from typing import TYPE_CHECKING, Any

import numpy as np
import torch

from setup.records import Record
from verification.commitment import merkle, native
from verification.commitment.encoding import (
    FLOAT_DTYPES,
    TAG_PRODUCT,
    TAG_WEIGHT,
    NonFiniteError,
    tensor_leaf_header,
    tensor_payload_span,
)
from verification.commitment.merkle import MerkleTree, hash_leaf, hash_record_leaf, merkle_root
from verification.transcript.errors import LeafDtypeError, LeafShapeError

if TYPE_CHECKING:
    from verification.computation.interface import DeclaredComputation

__all__ = [
    "leaf_parts", "leaf_hash", "leaf_hashes_of", "leaf_hashes_until_error", "leaf_hashes",
    "transcript_root", "commit_leaves", "hash_step_leaves", "HashStats", "leaf_totals",
    "dataset_tree", "dataset_root", "hash_step_leaves_device", "commit_leaves_device",
]

_NONFINITE = "float tensor contains NaN or Inf"
# A batch closes at this much host payload (which the library stages into HBM) or this many
# leaves; GPU-resident payloads are not counted.
_BATCH_HOST_BYTES = 4 << 30
_BATCH_ENTRIES = 1 << 20


class HashStats:
    """Where bulk hashing spent its time (seconds, accumulated across calls).

    ``read_s`` is the time inside the caller's item iterator, ``native_s`` the GPU calls
    (including their copies), ``producer_s`` the rest of the calling thread's work
    (validation, headers, batching). ``leaves`` and ``bytes`` count leaves and tensor payload
    bytes, ``batches`` the GPU calls.
    """

    __slots__ = ("read_s", "producer_s", "wait_s", "native_s", "big_s", "worker_other_s",
                 "batches", "leaves", "bytes")

    TIMES = ("read_s", "producer_s", "wait_s", "native_s", "big_s", "worker_other_s")

    def __init__(self) -> None:
        self.read_s = self.producer_s = self.wait_s = 0.0
        self.native_s = self.big_s = self.worker_other_s = 0.0
        self.batches = self.leaves = self.bytes = 0

    def times(self) -> dict[str, float]:
        return {k: getattr(self, k) for k in self.TIMES}

    def emit(self, section: Any, prefix: str) -> None:
        add = getattr(section, "add", None)
        if add is None:
            return
        for k in self.TIMES:
            v = getattr(self, k)
            if v > 0:
                add(f"{prefix}.{k.removesuffix('_s').removeprefix('worker_')}", v)


def _tensor_slot(c: DeclaredComputation,
                 index: int) -> tuple[int, tuple[int, ...], torch.dtype, str]:
    """``(tag, shape, dtype, slot name)`` of a non-record leaf."""
    n_s, n_w, M = c.n_s, c.n_w, c.M
    if n_s <= index < n_s + n_w:
        name = c.weight_names[index - n_s]
        return TAG_WEIGHT, tuple(c.weight_shapes[name]), c.weight_dtype, f"W_t[{name}]"
    if n_s + n_w <= index < n_s + n_w + M:
        spec = c.product(index - n_s - n_w + 1)
        return TAG_PRODUCT, spec.p_shape, c.product_dtype, f"P_{spec.m} ({spec.name})"
    if n_s + n_w + M <= index < c.n_leaves:
        name = c.weight_names[index - n_s - n_w - M]
        return TAG_WEIGHT, tuple(c.weight_shapes[name]), c.weight_dtype, f"W_t+1[{name}]"
    raise IndexError(f"leaf index {index} outside 0..{c.n_leaves - 1}")


def _checked_tensor(c: DeclaredComputation, index: int, obj: Any) -> tuple[int, torch.Tensor]:
    tag, shape, dtype, slot = _tensor_slot(c, index)
    if not isinstance(obj, torch.Tensor):
        raise LeafShapeError(f"leaf {index} {slot}: expected a tensor, got {type(obj).__name__}")
    if tuple(obj.shape) != shape:
        raise LeafShapeError(f"leaf {index} {slot}: shape {tuple(obj.shape)}, declared {shape}")
    if obj.dtype != dtype:
        raise LeafDtypeError(f"leaf {index} {slot}: dtype {obj.dtype}, declared {dtype}")
    return tag, obj


def leaf_parts(c: DeclaredComputation, index: int, obj: Any) -> tuple[bytes | memoryview, ...]:
    """Canonical bytes of leaf ``index`` holding ``obj``, as parts (host bytes)."""
    from verification.commitment.encoding import tensor_leaf_payload
    if 0 <= index < c.n_s:
        return (c.encode_record(obj),)
    tag, t = _checked_tensor(c, index, obj)
    return tensor_leaf_header(tag, t), tensor_leaf_payload(t)


def leaf_hash(c: DeclaredComputation, index: int, obj: Any) -> bytes:
    """``H_leaf`` of leaf ``index`` holding ``obj``."""
    return leaf_hashes_of(c, [(index, obj)])[0]


class _Batch:
    __slots__ = ("headers", "ptr", "nbytes", "kind", "keep", "host_bytes")

    def __init__(self) -> None:
        self.headers: list[bytes] = []
        self.ptr: list[int] = []
        self.nbytes: list[int] = []
        self.kind: list[int] = []
        self.keep: list[Any] = []
        self.host_bytes = 0


def _hash_batch(b: _Batch, stats: HashStats | None, plans: Any = None,
                site: str = "") -> tuple[list[bytes], int]:
    """One GPU call: the batch's digests and its first non-finite position (or its size).
    With ``plans`` (a verifier's plan cache) a batch whose payloads all lie in device memory
    runs the cached leaf plan of ``site`` when its layout is unchanged."""
    n = len(b.headers)
    if n == 0:
        return [], 0
    t0 = perf_counter()
    uniq: dict[bytes, int] = {}
    idx = np.empty(n, dtype=np.uint32)
    for i, h in enumerate(b.headers):
        idx[i] = uniq.setdefault(h, len(uniq))
    hdrs = list(uniq)
    hdr_len = np.array([len(h) for h in hdrs], dtype=np.uint32)
    hdr_off = np.zeros(len(hdrs), dtype=np.uint64)
    if len(hdrs) > 1:
        hdr_off[1:] = np.cumsum(hdr_len[:-1], dtype=np.uint64)
    ptr = np.array(b.ptr, dtype=np.uint64)
    nbytes = np.array(b.nbytes, dtype=np.uint64)
    kind = np.array(b.kind, dtype=np.uint8)
    if plans is not None and b.host_bytes == 0 and b.keep and \
            all(t.is_cuda for t in b.keep):
        dev = b.keep[0].device
        plan = plans.leaf_plan(site, b"".join(hdrs), hdr_off, hdr_len, idx, ptr, nbytes, kind,
                               dev)
        out, first_bad = plan.run()
        digests, bad = out.cpu().numpy(), int(first_bad.item())
    else:
        digests, bad = native.get().hash_leaves(b"".join(hdrs), hdr_off, hdr_len, idx, ptr,
                                                nbytes, kind)
    if stats is not None:
        stats.native_s += perf_counter() - t0
        stats.batches += 1
    raw = digests.tobytes()
    return [raw[32 * i:32 * i + 32] for i in range(min(bad, n))], bad


class _Slot:
    """What a tensor slot of ``C``'s layout requires, and its interned header."""

    __slots__ = ("tag", "shape", "dtype", "header", "kind")

    def __init__(self, tag: int, shape: tuple[int, ...], dtype: torch.dtype) -> None:
        self.tag, self.shape, self.dtype = tag, torch.Size(shape), dtype
        self.kind = native.FINITE_KIND.get(dtype)
        try:
            self.header: bytes | None = tensor_leaf_header(
                tag, torch.empty(shape, dtype=dtype, device="meta"))
        except Exception:  # an uncoded dtype: the slow path raises its error per leaf
            self.header = None


_SLOT_TABLES: weakref.WeakKeyDictionary[Any, list[_Slot]] = weakref.WeakKeyDictionary()


def _slot_table(c: DeclaredComputation) -> list[_Slot]:
    """The tensor slots of ``C`` (leaf ``n_s + j`` is entry ``j``), built once per
    computation: the layout of a declared computation does not change."""
    try:
        table = _SLOT_TABLES.get(c)
    except TypeError:  # not weakly referenceable: build it every time
        table = None
    if table is None or len(table) != c.n_leaves - c.n_s:
        table = [_Slot(*_tensor_slot(c, i)[:3]) for i in range(c.n_s, c.n_leaves)]
        try:
            _SLOT_TABLES[c] = table
        except TypeError:
            pass
    return table


def _until_error(c: DeclaredComputation, items: Iterable[tuple[int, Any]],
                 stats: HashStats | None, plans: Any = None,
                 site: str = "") -> tuple[list[bytes], Exception | None]:
    t_start = perf_counter()
    r0 = stats.read_s if stats is not None else 0.0
    n0 = stats.native_s if stats is not None else 0.0
    digests: list[bytes] = []
    batch = _Batch()
    finite_kind = native.FINITE_KIND
    hdr_cache: dict[tuple[int, torch.dtype, tuple[int, ...]], bytes] = {}
    error: Exception | None = None
    n_s = c.n_s
    table = _slot_table(c)
    n_table = len(table)
    tensor_type = torch.Tensor

    def flush() -> bool:
        nonlocal batch
        d, bad = _hash_batch(batch, stats, plans, site)
        digests.extend(d)
        ok = bad >= len(batch.headers)
        batch = _Batch()
        return ok

    records_open = False  # the batch holds records (a cached plan takes tensor leaves only)

    it = iter(items)
    try:
        while True:
            t0 = perf_counter()
            try:
                i, obj = next(it)
            except StopIteration:
                if stats is not None:
                    stats.read_s += perf_counter() - t0
                break
            if stats is not None:
                stats.read_s += perf_counter() - t0
                stats.leaves += 1
            if plans is not None:
                if 0 <= i < n_s:
                    records_open = True
                elif records_open:
                    records_open = False
                    if not flush():
                        return digests, NonFiniteError(_NONFINITE)
            try:
                j = i - n_s
                slot = table[j] if 0 <= j < n_table else None
                # The common case, a tensor leaf exactly as its slot declares, on the fast
                # path; anything else goes through the full validation, which raises the
                # reference's error for it.
                if (slot is not None and slot.header is not None and
                        isinstance(obj, tensor_type) and obj.dtype is slot.dtype and
                        obj.shape == slot.shape and obj.is_contiguous() and
                        (obj.is_cuda or obj.device.type == "cpu")):
                    t, h, kind = obj, slot.header, slot.kind
                else:
                    as_tensor = c.record_leaf(obj) if 0 <= i < n_s else None
                    if 0 <= i < n_s and as_tensor is None:
                        batch.headers.append(c.encode_record(obj))
                        batch.ptr.append(0)
                        batch.nbytes.append(0)
                        batch.kind.append(0)
                        t = None
                    else:
                        tag, t = as_tensor if as_tensor is not None \
                            else _checked_tensor(c, i, obj)
                        key = (tag, t.dtype, tuple(t.shape))
                        h = hdr_cache.get(key)
                        if h is None:
                            h = hdr_cache[key] = tensor_leaf_header(tag, t)
                        tensor_payload_span(t)  # the payload's own checks
                        kind = finite_kind[t.dtype]
                if t is not None:
                    nbytes = t.nbytes
                    batch.headers.append(h)
                    batch.ptr.append(t.data_ptr())
                    batch.nbytes.append(nbytes)
                    batch.kind.append(kind)
                    batch.keep.append(t)
                    if not t.is_cuda:
                        batch.host_bytes += nbytes
                    if stats is not None:
                        stats.bytes += nbytes
            except Exception as e:
                error = e
                break
            if batch.host_bytes >= _BATCH_HOST_BYTES or len(batch.headers) >= _BATCH_ENTRIES:
                if not flush():
                    return digests, NonFiniteError(_NONFINITE)
    except Exception as e:  # the iterator's own error; the leaves before it are still hashed
        error = e
    if not flush():
        return digests, NonFiniteError(_NONFINITE)
    if stats is not None:
        stats.producer_s += (perf_counter() - t_start - (stats.read_s - r0)
                             - (stats.native_s - n0))
    return digests, error


def leaf_hashes_of(c: DeclaredComputation, items: Iterable[tuple[int, Any]],
                   stats: HashStats | None = None, plans: Any = None,
                   site: str = "") -> list[bytes]:
    """The leaf hash of each ``(index, obj)`` in order; raises the first error a
    leaf-by-leaf loop raises. The objects must not change until this returns. ``plans`` (a
    verifier's plan cache) and ``site`` let device-resident leaves reuse the leaf plan of the
    same site's last call when their layout repeats."""
    digests, err = _until_error(c, items, stats, plans, site)
    if err is not None:
        raise err
    return digests


def leaf_hashes_until_error(c: DeclaredComputation, items: Iterable[tuple[int, Any]],
                            stats: HashStats | None = None, plans: Any = None,
                            site: str = "") -> tuple[list[bytes], Exception | None]:
    """:func:`leaf_hashes_of` up to the first error: ``(digests before it, error or None)``."""
    return _until_error(c, items, stats, plans, site)


def leaf_hashes(c: DeclaredComputation, reader: Any) -> list[bytes]:
    """Every leaf hash, from the reader's leaves over the declared ``n_leaves``."""
    return leaf_hashes_of(c, ((i, reader.leaf(i)) for i in range(c.n_leaves)))


def transcript_root(c: DeclaredComputation, reader: Any) -> bytes:
    """The root over the reader's leaves, never over supplied hashes."""
    return merkle_root(leaf_hashes(c, reader))


def hash_step_leaves(c: DeclaredComputation, leaves: Sequence[Any],
                     stats: HashStats | None = None) -> list[bytes]:
    """Every leaf hash of a full transcript, in layout order."""
    if len(leaves) != c.n_leaves:
        raise ValueError(f"transcript has {len(leaves)} leaves, the computation declares "
                         f"{c.n_leaves}")
    return leaf_hashes_of(c, enumerate(leaves), stats)


def commit_leaves(c: DeclaredComputation, leaves: Sequence[Any]) -> MerkleTree:
    """The Merkle tree over a full transcript; ``.root`` is ``h``."""
    return MerkleTree(hash_step_leaves(c, leaves))


def leaf_totals(c: DeclaredComputation, leaves: Sequence[Any]) -> tuple[int, int]:
    """``(leaf count, bytes)`` hashing counts: a record's encoding, a tensor's header and
    ``nbytes``."""
    total = 0
    for i, obj in enumerate(leaves):
        if i < c.n_s:
            total += len(c.encode_record(obj))
        else:
            total += len(tensor_leaf_header(_tensor_slot(c, i)[0], obj)) + obj.nbytes
    return len(leaves), total


def dataset_tree(c: DeclaredComputation, dataset: Sequence[Any]) -> MerkleTree:
    """The ``h_D`` tree over ``D``'s record leaves."""
    return MerkleTree(merkle.hash_leaves([(c.encode_record(r),) for r in dataset]))


def dataset_root(records: Sequence[Record]) -> bytes:
    """``h_D``: the Merkle root over the record leaves in record order."""
    return merkle_root([hash_record_leaf(r) for r in records])


# ---- GPU-resident transcripts -------------------------------------------------------------

class StepHasher:
    """A resident transcript's leaf-hashing plan: every leaf validated once, records staged
    in HBM, then :meth:`digests` enqueues the whole step's hashing with no host work."""

    def __init__(self, c: DeclaredComputation, leaves: Sequence[Any],
                 device: torch.device | None = None, fuse: Any = None) -> None:
        if len(leaves) != c.n_leaves:
            raise ValueError(f"transcript has {len(leaves)} leaves, the computation declares "
                             f"{c.n_leaves}")
        dev = device or next(t.device for t in leaves[c.n_s:] if isinstance(t, torch.Tensor))
        headers, payloads, kinds = [], [], []
        host_records: list[tuple[int, torch.Tensor]] = []
        record_headers: dict[tuple[int, torch.dtype, tuple[int, ...]], bytes] = {}
        for i, obj in enumerate(leaves):
            if i < c.n_s:
                as_tensor = c.record_leaf(obj)
                if as_tensor is not None:  # a tensor leaf: hashed where it lies
                    tag, t = as_tensor
                    key = (tag, t.dtype, tuple(t.shape))
                    if key not in record_headers:
                        record_headers[key] = tensor_leaf_header(tag, t)
                    headers.append(record_headers[key])
                    kinds.append(native.FINITE_KIND[t.dtype])
                    payloads.append(t if t.is_cuda else None)
                    if not t.is_cuda:
                        host_records.append((i, t))
                    continue
                rec = np.frombuffer(c.encode_record(obj), dtype=np.uint8).copy()
                headers.append(b"")
                payloads.append(torch.from_numpy(rec).to(dev))
                kinds.append(0)
                continue
            tag, t = _checked_tensor(c, i, obj)
            if not t.is_cuda:
                raise ValueError(f"leaf {i} is not on the GPU")
            headers.append(tensor_leaf_header(tag, t))
            payloads.append(t)
            kinds.append(native.FINITE_KIND[t.dtype])
        if host_records:  # one copy to the device for every host record tensor
            flat = torch.cat([t.contiguous().view(-1).view(torch.uint8)
                              for _, t in host_records]).to(dev)
            self._records = flat
            o = 0
            for i, t in host_records:
                n = t.numel() * t.element_size()
                payloads[i] = flat[o:o + n].view(t.dtype).view(t.shape)
                o += n
        self.c = c
        # With `fuse` (a native.FvPlan over this step's products), the product leaves' P-pass
        # sums are taken while they are hashed.
        self.plan = native.get().leaf_plan(headers, payloads, kinds, fuse)
        self.n = len(leaves)
        self.bytes = self.plan.bytes

    def digests(self, out: torch.Tensor | None = None, bad: torch.Tensor | None = None,
                stream: torch.cuda.Stream | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """``(digests uint8 [n, 32], first_bad int32 [1])`` on the GPU, stream-ordered."""
        return self.plan.run(out, bad, stream)


def hash_step_leaves_device(c: DeclaredComputation, leaves: Sequence[Any]) -> torch.Tensor:
    """Every leaf hash of a GPU-resident transcript, uint8 ``[n_leaves, 32]`` in HBM. Raises
    ``NonFiniteError`` if a float leaf holds NaN or Inf."""
    d, bad = StepHasher(c, leaves).digests()
    if int(bad.item()) < len(leaves):
        raise NonFiniteError(_NONFINITE)
    return d


def commit_leaves_device(c: DeclaredComputation, leaves: Sequence[Any]) -> MerkleTree:
    """:func:`commit_leaves` for a GPU-resident transcript: hashing and tree on the GPU."""
    d = hash_step_leaves_device(c, leaves)
    nodes = native.get().merkle_tree_device(d)
    return MerkleTree.from_nodes(nodes.cpu().numpy().tobytes(), d.shape[0])
