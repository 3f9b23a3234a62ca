"""A stored step brought into device memory in one pass.

The reference reads its on-disk store one file at a time (verification/transcript/store.py
:347-357, ``DiskStore.leaf``): ``torch.load`` into pageable host memory, after which each check
copies what it needs to the GPU. :func:`load_step` moves a whole step instead, natively:

1. ``pots_store_scan`` reads every leaf file's ZIP directory and pickle on host threads. For a
   file that holds one plain tensor it returns the dtype, shape, strides, storage offset and
   the place of the storage's bytes in the file; nothing is unpickled or executed.
2. The step's storages are laid out end to end in one device buffer (the arena), each at a
   256-byte aligned offset, in leaf order.
3. ``pots_store_load`` reads the bytes with ``pread`` on host threads into pinned staging
   slots and sends each filled slot to the arena with one DMA copy.
4. Each leaf becomes a tensor over its part of the arena (``Tensor.set_``: every leaf keeps a
   version counter of its own).

A file the scan does not take is read with :meth:`DiskStore.leaf` itself, i.e.
``torch.load(weights_only=True)`` and its error mapping. Records (the ``{"ids", "mask",
"targets"}`` dicts) stay on the host, where the verifier encodes them; any other such tensor is
copied into the arena after the native load. A file that fails to read keeps its exception,
and :class:`ResidentStore` raises it when that leaf is read, so the verifier rejects at the
first bad leaf in order as it does over a :class:`DiskStore`.

The leaves equal ``[store.leaf(i) for i in range(n)]`` bit for bit, with the same dtypes,
shapes, strides and storage offsets, on the device.

Captured operands (``A_m``, ``B_m`` of every product) are not part of the reference's store:
its verifier replays the model to get them. This build has no replay, so a stored step that
is to be verified keeps the operands the prover used in ``operands/op_{m:05d}_{a|b}.pt``
beside the leaf files (:func:`write_operands`); :func:`load_step` brings them in with the
leaves.
"""

from __future__ import annotations

import ctypes
import os
import threading
import time
from collections.abc import Mapping, Sequence
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import numpy as np
import torch

from verification.commitment import native
from verification.transcript.errors import LeafReadError, StoreMutationError
from verification.transcript.store import (LEAF_FILE, DiskStore, TranscriptStore, _versions,
                                           savable)

__all__ = ["ALIGN", "OPERAND_DIR", "OPERAND_FILE", "STORE_DTYPES", "StoredStep",
           "ResidentStore", "StepLoader", "load_step", "scan_files", "write_operands"]

ALIGN = 256
OPERAND_DIR = "operands"
OPERAND_FILE = "op_{:05d}_{}.pt"

STORE_OK, STORE_OTHER, STORE_UNREADABLE = 0, 1, 2
STORE_DTYPES: dict[int, torch.dtype] = {
    1: torch.float32, 2: torch.float64, 3: torch.float16, 4: torch.bfloat16, 5: torch.int64,
    6: torch.int32, 7: torch.int16, 8: torch.int8, 9: torch.uint8, 10: torch.bool,
}

_STORED = np.dtype([("data_offset", "<u8"), ("storage_bytes", "<u8"), ("storage_offset", "<u8"),
                    ("size", "<i8", (8,)), ("stride", "<i8", (8,)), ("ndim", "<u4"),
                    ("dtype", "<u4"), ("status", "<i4"), ("pad", "<u4")])
_SEGMENT = np.dtype([("file", "<u4"), ("pad", "<u4"), ("file_offset", "<u8"), ("bytes", "<u8"),
                     ("dst_offset", "<u8")])
assert _STORED.itemsize == 168 and _SEGMENT.itemsize == 32

_LIB = None
_LIB_LOCK = threading.Lock()


def _lib() -> ctypes.CDLL:
    """The library's host-side store entry points (they need no GPU: the scan, and loads into
    host memory)."""
    global _LIB
    with _LIB_LOCK:
        if _LIB is None:
            if not native.LIB_PATH.exists():
                raise RuntimeError(f"{native.LIB_PATH} is missing: build it with "
                                   "`python pots-2.0_amd/build.py` (hipcc, gfx950)")
            lib = ctypes.CDLL(str(native.LIB_PATH))
            vp, u32, u64, i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int
            lib.pots_store_scan.argtypes = [u32, vp, vp, u32]
            lib.pots_store_scan.restype = i32
            lib.pots_store_load.argtypes = [u32, vp, u32, vp, vp, i32, vp, u64, u32]
            lib.pots_store_load.restype = i32
            lib.pots_last_error.argtypes = []
            lib.pots_last_error.restype = ctypes.c_char_p
            _LIB = lib
        return _LIB


def _check(rc: int, what: str) -> None:
    if rc == native.E_OK:
        return
    if rc == native.E_ARG:
        raise ValueError(f"{what}: argument rejected by libpots_mi355x")
    msg = _lib().pots_last_error().decode(errors="replace")
    if rc == native.E_IO:
        raise LeafReadError(f"{what}: {msg}")
    raise native.NativeError(f"{what} failed with {rc}: {msg}")


class _PathTable:
    """File names as the C ABI takes them: an array of pointers to NUL-terminated bytes, built
    with numpy (a step has tens of thousands of files)."""

    def __init__(self, paths: Sequence[str | bytes | os.PathLike]) -> None:
        raw = [p if isinstance(p, bytes) else os.fsencode(p) for p in paths]
        self.raw = raw
        self.buf = np.frombuffer(b"\0".join(raw) + b"\0", dtype=np.uint8)
        lens = np.fromiter((len(r) + 1 for r in raw), dtype=np.uint64, count=len(raw))
        starts = np.zeros(len(raw), dtype=np.uint64)
        if len(raw) > 1:
            np.cumsum(lens[:-1], out=starts[1:])
        self.ptrs = starts + np.uint64(self.buf.ctypes.data)

    def __len__(self) -> int:
        return len(self.raw)

    @property
    def address(self) -> int:
        return self.ptrs.ctypes.data

    def path(self, k: int) -> Path:
        return Path(os.fsdecode(self.raw[k]))


def scan_files(paths: Sequence[str | bytes | os.PathLike] | _PathTable, threads: int = 0
               ) -> np.ndarray:
    """``pots_store_scan`` over ``paths``: one structured record per file."""
    table = paths if isinstance(paths, _PathTable) else _PathTable(paths)
    out = np.zeros(len(table), dtype=_STORED)
    if not len(table):
        return out
    _check(_lib().pots_store_scan(len(table), table.address, out.ctypes.data, threads),
           "pots_store_scan")
    return out


def write_operands(directory: str | Path, operands: Mapping[int, tuple[torch.Tensor,
                                                                      torch.Tensor]]) -> None:
    """Store each product's captured ``(A_m, B_m)`` under ``directory/operands``."""
    d = Path(directory) / OPERAND_DIR
    d.mkdir(parents=True, exist_ok=True)
    for m, (a, b) in operands.items():
        torch.save(savable(a), d / OPERAND_FILE.format(m, "a"))
        torch.save(savable(b), d / OPERAND_FILE.format(m, "b"))


@dataclass
class StoredStep:
    """A stored step in device memory: its leaves (an exception in place of each leaf that
    failed to read), the captured operands asked for, and what the load cost."""

    leaves: list[Any]
    operands: dict[int, tuple[torch.Tensor, torch.Tensor]]
    arena: torch.Tensor
    bytes: int                   # storage bytes moved by the native load
    files: int
    fallback: int                # files read with torch.load
    times: dict[str, float] = field(default_factory=dict)


class ResidentStore(TranscriptStore):
    """The verifier's view of a step :func:`load_step` brought in: leaves from the arena (a
    leaf that failed to read raises its error again), root and paths from the directory."""

    def __init__(self, disk: DiskStore, step: StoredStep) -> None:
        self.disk, self.step = disk, step
        self._versions = [None if isinstance(x, BaseException) else _versions(x)
                          for x in step.leaves]

    def leaf(self, index: int) -> Any:
        if not isinstance(index, int) or not 0 <= index < len(self.step.leaves):
            raise IndexError(f"leaf index {index!r} out of range")
        obj = self.step.leaves[index]
        if isinstance(obj, BaseException):
            raise obj
        if _versions(obj) != self._versions[index]:
            raise StoreMutationError(f"leaf {index} changed in place after the load")
        return obj

    @property
    def root(self) -> bytes:
        return self.disk.root

    def path(self, index: int) -> list[bytes]:
        return self.disk.path(index)

    def dataset_path(self, i: int) -> list[bytes]:
        return self.disk.dataset_path(i)


def _aligned(n: int) -> int:
    return (n + ALIGN - 1) // ALIGN * ALIGN


_ESZ = {dt: torch.empty(0, dtype=dt).element_size() for dt in STORE_DTYPES.values()}


class _Views:
    """Tensors over one arena, each with a version counter of its own (``Tensor.set_`` on a
    fresh tensor, not a view of the arena)."""

    def __init__(self, arena: torch.Tensor) -> None:
        self.storage = arena.untyped_storage()
        self.base = arena.storage_offset()
        self.device = arena.device
        self.empty = {dt: torch.empty(0, dtype=dt, device=arena.device)
                      for dt in STORE_DTYPES.values()}

    def __call__(self, off: int, dtype: torch.dtype, size: Sequence[int],
                 stride: Sequence[int], storage_offset: int) -> torch.Tensor:
        t = self.empty[dtype].new_empty(0) if dtype in self.empty else \
            torch.empty(0, dtype=dtype, device=self.device)
        esz = t.element_size()
        return t.set_(self.storage, (self.base + off) // esz + storage_offset, size, stride)


def _bytes_of(t: torch.Tensor) -> torch.Tensor:
    """The whole storage of host tensor ``t`` as uint8."""
    st = t.untyped_storage()
    return torch.empty(0, dtype=torch.uint8).set_(st, 0, (st.nbytes(),), (1,))


class StepLoader:
    """Loads stored steps to one device, reusing its pinned staging (``staging_mib`` MiB,
    two slots per thread) across loads. ``device`` ``cpu`` loads into host memory."""

    def __init__(self, device: torch.device | str | None = None, *, threads: int = 8,
                 staging_mib: int = 256) -> None:
        if device is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.threads = max(1, min(64, int(threads)))
        self.staging = None
        if self.device.type == "cuda":
            self.staging = torch.empty(int(staging_mib) << 20, dtype=torch.uint8,
                                       pin_memory=True)

    def load(self, store: DiskStore, n_leaves: int, operand_ms: Sequence[int] = ()
             ) -> StoredStep:
        """Leaves ``0 .. n_leaves-1`` of ``store`` (the count comes from the computation, not
        the store) and the captured operands of products ``operand_ms``."""
        times: dict[str, float] = {}
        t0 = time.perf_counter()
        d = os.fsencode(store.directory)
        leaf_name = os.fsencode(LEAF_FILE).replace(b"{:05d}", b"%05d")
        op_name = os.fsencode(f"{OPERAND_DIR}/{OPERAND_FILE}").replace(b"{:05d}_{}", b"%05d_%s")
        paths = _PathTable([d + b"/" + leaf_name % i for i in range(n_leaves)] +
                           [d + b"/" + op_name % (m, w) for m in operand_ms for w in (b"a", b"b")])
        info = scan_files(paths, self.threads)
        times["scan"] = time.perf_counter() - t0

        # Layout: every scanned storage, then every fallback tensor's storage.
        t1 = time.perf_counter()
        offsets = np.zeros(len(paths), dtype=np.int64)
        ok = info["status"] == STORE_OK
        aligned = (info["storage_bytes"][ok].astype(np.int64) + ALIGN - 1) // ALIGN * ALIGN
        ends = np.cumsum(aligned)
        offsets[ok] = ends - aligned
        off = int(ends[-1]) if len(ends) else 0
        objs: dict[int, Any] = {}
        fb_tensors: list[tuple[int, torch.Tensor]] = []
        for k in np.flatnonzero(~ok):
            k = int(k)
            try:
                if k < n_leaves:
                    obj = store.leaf(k)
                else:
                    try:
                        obj = torch.load(paths.path(k), map_location="cpu",
                                         weights_only=True)
                    except Exception as e:
                        raise LeafReadError(f"operand file {paths.path(k).name} unreadable: "
                                            f"{type(e).__name__}: {e}") from e
                    if not isinstance(obj, torch.Tensor):
                        raise LeafReadError(f"operand file {paths.path(k).name} holds no "
                                            "tensor")
            except Exception as e:  # kept, and raised when the leaf is read
                if k >= n_leaves:
                    raise
                objs[k] = e
                continue
            objs[k] = obj
            if isinstance(obj, torch.Tensor):
                offsets[k] = off
                off += _aligned(obj.untyped_storage().nbytes())
                fb_tensors.append((k, obj))
        times["fallback_read"] = time.perf_counter() - t1

        t2 = time.perf_counter()
        arena = torch.empty(max(off, ALIGN), dtype=torch.uint8, device=self.device)
        segs = np.zeros(int(ok.sum()), dtype=_SEGMENT)
        idx = np.flatnonzero(ok)
        segs["file"] = idx
        segs["file_offset"] = info["data_offset"][idx]
        segs["bytes"] = info["storage_bytes"][idx]
        segs["dst_offset"] = offsets[idx]
        moved = int(segs["bytes"].sum())
        # The native load runs on a thread of its own (ctypes lets go of the GIL), while this
        # thread lays the leaves' tensors over the arena: they need only the offsets.
        failure: list[BaseException] = []
        native_s = [0.0]

        def native_load() -> None:
            t = time.perf_counter()
            try:
                host = self.device.type != "cuda"
                staging = 0 if host else self.staging.data_ptr()
                staging_bytes = 0 if host else self.staging.numel()
                _check(_lib().pots_store_load(
                    len(paths), paths.address, len(segs), segs.ctypes.data,
                    arena.data_ptr(), -1 if host else self.device.index, staging,
                    staging_bytes, self.threads), "pots_store_load")
            except BaseException as e:  # raised on the caller's thread below
                failure.append(e)
            native_s[0] = time.perf_counter() - t

        worker = threading.Thread(target=native_load, name="pots-store-load")
        if len(segs):
            worker.start()
        t3 = time.perf_counter()
        view = _Views(arena)
        out: list[Any] = []
        cols = (ok.tolist(), offsets.tolist(), info["dtype"].tolist(), info["ndim"].tolist(),
                info["size"].tolist(), info["stride"].tolist(), info["storage_offset"].tolist())
        for k, (good, o, dt, nd, size, stride, so) in enumerate(zip(*cols)):
            if good:
                v = view(o, STORE_DTYPES[dt], size[:nd], stride[:nd], so)
            else:
                v = objs[k]
                if isinstance(v, torch.Tensor):
                    t = v
                    v = view(o, t.dtype, t.shape, t.stride(), t.storage_offset())
                    if t.requires_grad:
                        v.requires_grad_(True)
            out.append(v)
        times["build"] = time.perf_counter() - t3
        if len(segs):
            worker.join()
        times["load"] = native_s[0]
        times["load_and_build"] = time.perf_counter() - t2
        if failure:
            raise failure[0]
        # Fallback tensors after the native load: its spans may write the bytes between
        # segments.
        for k, t in fb_tensors:
            nb = t.untyped_storage().nbytes()
            if nb:
                o = int(offsets[k])
                arena[o:o + nb].copy_(_bytes_of(t))
        if self.device.type == "cuda":
            torch.cuda.current_stream(self.device).synchronize()
        leaves = out[:n_leaves]
        ops = {m: (out[n_leaves + 2 * j], out[n_leaves + 2 * j + 1])
               for j, m in enumerate(operand_ms)}
        return StoredStep(leaves, ops, arena, moved, len(paths), len(objs), times)


def load_step(store: DiskStore | str | Path, n_leaves: int, device: torch.device | str | None
              = None, *, operand_ms: Sequence[int] = (), threads: int = 8,
              staging_mib: int = 256) -> StoredStep:
    """:meth:`StepLoader.load` with a loader of its own."""
    if not isinstance(store, DiskStore):
        store = DiskStore(store)
    return StepLoader(device, threads=threads, staging_mib=staging_mib).load(
        store, n_leaves, operand_ms)
