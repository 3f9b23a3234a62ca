"""The on-disk transcript store and its native reader, on the host (no GPU needed).

The store's tests follow the reference's (tests/verification/transcript/test_store.py:306-426):
a round trip in the reference's file layout, fresh reads that share nothing, a view saved as
itself, bad files as prover-data errors, a write that replaces or cleans up, and the
hand-offs. The reader's tests pin ``pots_store_scan`` and ``pots_store_load`` against
``torch.load`` itself: every file the scan takes must load to the same dtype, shape, strides,
storage offset and bytes; everything else must be left to ``torch.load`` (status OTHER or
UNREADABLE). Merkle trees are built from the CPU oracle's node buffer, since the library's
hashing needs a GPU.
"""

from __future__ import annotations

import json
import random
import struct
import zipfile
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as O
from setup.records import Record, RecordError
from verification.commitment.merkle import MerkleTree
from verification.transcript import loader as L
from verification.transcript.errors import LeafReadError, StoreMutationError
from verification.transcript.store import (DISK_FORMAT, HASHES_FILE, IN_MEMORY, LEAF_FILE,
                                           META_FILE, DiskHandoff, DiskStore, InMemoryStore,
                                           disk_object)


class _C:
    n_s = 2


def _record(n, seed):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, 1000, (n,), generator=g, dtype=torch.int32)
    return Record(ids, torch.roll(ids, -1), torch.ones(n, dtype=torch.int32))


def _leaves():
    g = torch.Generator().manual_seed(5)
    base = torch.arange(40, dtype=torch.float32).reshape(5, 8)
    return [_record(9, 1), _record(4, 2),
            torch.randn(33, 17, generator=g),
            torch.randn(7, 300, generator=g).to(torch.bfloat16),
            base[1:3],
            torch.randn(64, 48, generator=g),
            torch.randn(48, generator=g)]


def _tree(n, seed=0):
    rng = np.random.default_rng(seed)
    hashes = [bytes(rng.integers(0, 256, 32, dtype=np.uint8)) for _ in range(n)]
    return MerkleTree.from_nodes(O.merkle_tree(hashes), n)


def _paths(n, seed=1):
    rng = np.random.default_rng(seed)
    return [[bytes(rng.integers(0, 256, 32, dtype=np.uint8)) for _ in range(3)]
            for _ in range(n)]


def _same(a, b):
    if isinstance(a, torch.Tensor):
        return (isinstance(b, torch.Tensor) and a.dtype == b.dtype and a.shape == b.shape
                and torch.equal(a.detach().cpu(), b.detach().cpu()))
    return isinstance(b, Record) and all(_same(getattr(a, k), getattr(b, k))
                                         for k in ("ids", "targets", "mask"))


def _write(tmp_path, leaves=None, paths=True):
    leaves = _leaves() if leaves is None else leaves
    tree = _tree(len(leaves))
    dp = _paths(_C.n_s) if paths else None
    return leaves, tree, dp, DiskStore.write(tmp_path / "step", _C, leaves, tree, dp)


# ---- the store --------------------------------------------------------------------------


def test_disk_store_round_trip(tmp_path):
    leaves, tree, dp, disk = _write(tmp_path)
    assert disk.root == tree.root
    for i, obj in enumerate(leaves):
        assert _same(obj, disk.leaf(i))
    assert disk.leaf_hashes() == [tree.leaf(i) for i in range(len(leaves))]
    for i in range(_C.n_s):
        assert disk.dataset_path(i) == dp[i]
    assert sorted(p.name for p in disk.directory.iterdir()) == sorted(
        [LEAF_FILE.format(i) for i in range(len(leaves))] + [META_FILE, HASHES_FILE])
    meta = json.loads((disk.directory / META_FILE).read_text())
    assert meta == {"format": DISK_FORMAT, "root": tree.root.hex(),
                    "dataset_paths": [[h.hex() for h in p] for p in dp]}
    # A record is saved as the reference saves it: a dict of its three int32 tensors.
    rec = torch.load(disk.leaf_path(0), weights_only=True)
    assert sorted(rec) == ["ids", "mask", "targets"]


def test_disk_reads_are_fresh_and_share_nothing(tmp_path):
    leaves, _, _, disk = _write(tmp_path)
    a, b = disk.leaf(2), disk.leaf(2)
    assert a is not b and a.untyped_storage().data_ptr() != b.untyped_storage().data_ptr()
    a.add_(1.0)  # a reader's write reaches neither the file nor the next read
    assert _same(disk.leaf(2), leaves[2])


def test_disk_write_of_a_view_saves_only_the_view(tmp_path):
    base = torch.arange(40, dtype=torch.float32).reshape(5, 8)
    torch.save(disk_object(base[1:3]), tmp_path / "v.pt")
    torch.save(disk_object(base), tmp_path / "b.pt")
    assert (tmp_path / "v.pt").stat().st_size < (tmp_path / "b.pt").stat().st_size
    assert torch.equal(torch.load(tmp_path / "v.pt", weights_only=True), base[1:3])


def test_disk_store_bad_files_are_prover_data_errors(tmp_path):
    _, _, _, disk = _write(tmp_path)
    d = disk.directory
    with pytest.raises(IndexError):
        disk.leaf(7)  # no such file
    with pytest.raises(IndexError):
        disk.leaf(-1)
    (d / LEAF_FILE.format(3)).write_bytes(b"not a torch file")
    with pytest.raises(LeafReadError):
        disk.leaf(3)
    torch.save({"x": torch.zeros(2)}, d / LEAF_FILE.format(5))
    with pytest.raises(LeafReadError):
        disk.leaf(5)
    torch.save({"ids": torch.zeros(3, dtype=torch.int64), "targets": torch.zeros(3),
                "mask": torch.zeros(3)}, d / LEAF_FILE.format(0))
    with pytest.raises(RecordError):
        disk.leaf(0)
    (d / LEAF_FILE.format(6)).unlink()
    with pytest.raises(IndexError):
        disk.leaf(6)
    (d / HASHES_FILE).write_bytes(b"\0" * 33)
    with pytest.raises(LeafReadError):
        disk.leaf_hashes()
    (d / META_FILE).unlink()
    with pytest.raises(LeafReadError):
        _ = disk.root
    with pytest.raises(LeafReadError):
        disk.dataset_path(0)
    (d / META_FILE).write_text(json.dumps({"format": 2, "root": "00" * 32}))
    with pytest.raises(LeafReadError):
        _ = disk.root
    assert issubclass(LeafReadError, ValueError)  # so the verifier's guard maps it


def test_disk_store_without_dataset_paths(tmp_path):
    _, _, _, disk = _write(tmp_path, paths=False)
    with pytest.raises(LookupError):
        disk.dataset_path(0)


def test_disk_write_replaces_and_failed_write_cleans_up(tmp_path):
    d = tmp_path / "step"
    d.mkdir()
    (d / "stale").write_text("x")
    leaves, tree, _, _ = _write(tmp_path)
    assert not (d / "stale").exists()
    with pytest.raises(TypeError):
        DiskStore.write(d, _C, [*leaves[:-1], object()], tree)
    assert not d.exists()
    with pytest.raises(ValueError):
        DiskStore.write(d, _C, leaves[:-1], tree)
    with pytest.raises(ValueError):
        DiskStore.write(d, _C, leaves, tree, _paths(3))


def test_handoffs(tmp_path):
    leaves = _leaves()
    tree = _tree(len(leaves))
    h = DiskHandoff(tmp_path / "run")
    store = h.hold(_C, 3, leaves, tree)
    assert isinstance(store, DiskStore) and store.directory == tmp_path / "run" / "step_3"
    assert store.root == tree.root
    h.release(store)
    assert not (tmp_path / "run" / "step_3").exists()
    keep = DiskHandoff(tmp_path / "run", keep=True)
    s2 = keep.hold(_C, 1, leaves, tree)
    keep.release(s2)
    assert s2.directory.exists()
    mem = IN_MEMORY.hold(_C, 1, leaves, tree)
    assert isinstance(mem, InMemoryStore) and mem.root == tree.root
    IN_MEMORY.release(mem)


# ---- pots_store_scan against torch.load --------------------------------------------------


def _storage_bytes(t: torch.Tensor) -> bytes:
    st = t.untyped_storage()
    return bytes(torch.empty(0, dtype=torch.uint8).set_(st, 0, (st.nbytes(),), (1,)).numpy())


def _agrees(path: Path, r) -> None:
    """A file the scan took loads with torch.load to exactly what the scan describes."""
    t = torch.load(path, map_location="cpu", weights_only=True)
    assert isinstance(t, torch.Tensor) and not t.requires_grad
    nd = int(r["ndim"])
    assert L.STORE_DTYPES[int(r["dtype"])] == t.dtype
    assert r["size"][:nd].tolist() == list(t.shape)
    assert r["stride"][:nd].tolist() == list(t.stride())
    assert int(r["storage_offset"]) == t.storage_offset()
    assert int(r["storage_bytes"]) == t.untyped_storage().nbytes()
    with open(path, "rb") as f:
        f.seek(int(r["data_offset"]))
        assert f.read(int(r["storage_bytes"])) == _storage_bytes(t)


def test_scan_takes_every_plain_tensor(tmp_path):
    g = torch.Generator().manual_seed(0)
    cases = [torch.randn(3, 5, generator=g).to(dt) for dt in
             (torch.float32, torch.float64, torch.float16, torch.bfloat16)]
    cases += [torch.randint(-100, 100, (4, 6), generator=g, dtype=dt) for dt in
              (torch.int64, torch.int32, torch.int16, torch.int8)]
    cases += [torch.randint(0, 255, (7,), generator=g, dtype=torch.uint8),
              torch.rand(9, generator=g) > 0.5, torch.tensor(2.5),
              torch.randn(2, 3, 4, 5, generator=g).permute(3, 1, 0, 2),  # owns its storage
              torch.arange(40.0).reshape(5, 8)[1:3, 2:6],                  # a raw view
              torch.randn(300, 700, generator=g)]
    paths = []
    for i, t in enumerate(cases):
        p = tmp_path / f"t{i}.pt"
        torch.save(t, p)
        paths.append(p)
    info = L.scan_files(paths, threads=3)
    assert (info["status"] == L.STORE_OK).all(), info["status"]
    for p, r in zip(paths, info):
        _agrees(p, r)
    raw_view = info[len(cases) - 2]
    assert int(raw_view["storage_offset"]) == 10 and int(raw_view["storage_bytes"]) == 160


def test_scan_leaves_everything_else_to_torch_load(tmp_path):
    objs = {"record": {"ids": torch.zeros(3, dtype=torch.int32),
                       "mask": torch.ones(3, dtype=torch.int32),
                       "targets": torch.zeros(3, dtype=torch.int32)},
            "grad": torch.randn(3, requires_grad=True),
            "empty": torch.zeros(0, 4),
            "pair": (torch.zeros(2), torch.ones(2)),
            "list": [torch.zeros(2)],
            "int": 7}
    paths = []
    for name, obj in objs.items():
        torch.save(obj, tmp_path / f"{name}.pt")
        paths.append(tmp_path / f"{name}.pt")
    (tmp_path / "junk.pt").write_bytes(b"not a torch file")
    (tmp_path / "short.pt").write_bytes(b"PK")
    paths += [tmp_path / "junk.pt", tmp_path / "short.pt", tmp_path / "missing.pt", tmp_path]
    info = L.scan_files(paths)
    assert info["status"].tolist() == [L.STORE_OTHER] * len(objs) + [L.STORE_UNREADABLE] * 4


def _repack(src: Path, dst: Path, **kw) -> None:
    """The records of a torch.save file in a ZIP written by Python's zipfile."""
    with zipfile.ZipFile(src) as zin, zipfile.ZipFile(dst, "w", zipfile.ZIP_STORED) as zout:
        for info in zin.infolist():
            data = zin.read(info)
            with zout.open(zipfile.ZipInfo(info.filename), "w", **kw) as f:
                f.write(data)


def test_scan_reads_zip64_archives(tmp_path, monkeypatch):
    """ZIP64 records as an archive over 4 GiB has them: zipfile's limits lowered so that
    every size and offset past 100 bytes, and the directory's end, take their ZIP64 form."""
    t = torch.randn(50, 60)
    torch.save(t, tmp_path / "a.pt")
    monkeypatch.setattr(zipfile, "ZIP64_LIMIT", 100)
    monkeypatch.setattr(zipfile, "ZIP_FILECOUNT_LIMIT", 2)
    _repack(tmp_path / "a.pt", tmp_path / "z.pt", force_zip64=True)
    monkeypatch.undo()
    raw = (tmp_path / "z.pt").read_bytes()
    assert b"PK\x06\x06" in raw and b"PK\x06\x07" in raw  # ZIP64 end record and locator
    with zipfile.ZipFile(tmp_path / "z.pt") as zf:
        data = next(i for i in zf.infolist() if "/data/" in i.filename)
        assert data.extra[:2] == b"\x01\x00"  # the ZIP64 extended information field
    assert torch.equal(torch.load(tmp_path / "z.pt", weights_only=True), t)
    (r,) = L.scan_files([tmp_path / "z.pt"])
    assert r["status"] == L.STORE_OK
    _agrees(tmp_path / "z.pt", r)


def test_scan_refuses_big_endian_and_compressed_archives(tmp_path):
    t = torch.randn(8, 8)
    torch.save(t, tmp_path / "a.pt")
    with zipfile.ZipFile(tmp_path / "a.pt") as zin, \
            zipfile.ZipFile(tmp_path / "big.pt", "w", zipfile.ZIP_STORED) as zout:
        for info in zin.infolist():
            data = zin.read(info)
            zout.writestr(info.filename, b"big" if info.filename.endswith("/byteorder")
                          else data)
    with zipfile.ZipFile(tmp_path / "a.pt") as zin, \
            zipfile.ZipFile(tmp_path / "deflated.pt", "w", zipfile.ZIP_DEFLATED) as zout:
        for info in zin.infolist():
            zout.writestr(info.filename, zin.read(info))
    info = L.scan_files([tmp_path / "big.pt", tmp_path / "deflated.pt"])
    assert info["status"].tolist() == [L.STORE_OTHER, L.STORE_OTHER]


def _record_span(raw: bytes, info: zipfile.ZipInfo) -> tuple[int, int]:
    nl, xl = struct.unpack("<HH", raw[info.header_offset + 26:info.header_offset + 30])
    lo = info.header_offset + 30 + nl + xl
    return lo, lo + info.file_size


@pytest.mark.filterwarnings("ignore:Detected pickle protocol")
@pytest.mark.parametrize("region", ["archive", "pickle"])
@pytest.mark.parametrize("tensor", ["f32", "bf16_permuted"])
def test_scan_never_takes_a_damaged_file_torch_load_reads_otherwise(tmp_path, region, tensor):
    """Bytes changed anywhere in the archive (or only in the pickle): whenever the scan still
    takes the file, torch.load reads it to exactly what the scan describes."""
    t = (torch.arange(60, dtype=torch.float32).reshape(6, 10) if tensor == "f32" else
         torch.randn(3, 4, 50, generator=torch.Generator().manual_seed(0))
         .to(torch.bfloat16).permute(2, 0, 1))
    torch.save(t, tmp_path / "a.pt")
    raw = (tmp_path / "a.pt").read_bytes()
    with zipfile.ZipFile(tmp_path / "a.pt") as zf:
        data_lo, data_hi = _record_span(raw, next(i for i in zf.infolist()
                                                  if "/data/" in i.filename))
        pk_lo, pk_hi = _record_span(raw, next(i for i in zf.infolist()
                                              if i.filename.endswith("/data.pkl")))
    rng = random.Random({"archive": 7, "pickle": 11}[region] + 100 * (tensor == "f32"))
    paths = []
    for k in range(300):
        b = bytearray(raw)
        for _ in range(rng.choice((1, 1, 2, 3, 5))):
            while True:
                pos = rng.randrange(pk_lo, pk_hi) if region == "pickle" else \
                    rng.randrange(len(b))
                if not data_lo <= pos < data_hi:  # the values themselves are free bytes
                    break
            b[pos] = rng.randrange(256)
        p = tmp_path / f"f{k}.pt"
        p.write_bytes(bytes(b))
        paths.append(p)
    info = L.scan_files(paths, threads=4)
    taken = 0
    for p, r in zip(paths, info):
        if r["status"] == L.STORE_OK:
            taken += 1
            _agrees(p, r)
    assert 0 < taken < len(paths)


def test_scan_refuses_a_memo_put_with_nothing_to_memoize(tmp_path):
    """A pickle that opens with BINPUT: torch.load fails on it (the unpickler's stack is
    empty), so the scan must not take it."""
    torch.save(torch.zeros(4), tmp_path / "a.pt")
    raw = bytearray((tmp_path / "a.pt").read_bytes())
    with zipfile.ZipFile(tmp_path / "a.pt") as zf:
        lo, _ = _record_span(bytes(raw), next(i for i in zf.infolist()
                                              if i.filename.endswith("/data.pkl")))
    assert raw[lo] == 0x80  # PROTO
    raw[lo] = ord("q")      # BINPUT 2
    (tmp_path / "b.pt").write_bytes(bytes(raw))
    with pytest.raises(Exception):
        torch.load(tmp_path / "b.pt", weights_only=True)
    assert L.scan_files([tmp_path / "b.pt"])["status"][0] == L.STORE_OTHER


# ---- pots_store_load and the loader on the host ------------------------------------------


def test_loader_equals_disk_reads_on_the_host(tmp_path):
    leaves = _leaves() + [torch.randn(3), torch.zeros(0, 4), torch.randn(1000, 700)]
    _, _, _, disk = _write(tmp_path, leaves)
    # A prover's file may hold a tensor that needs grad (the store's own writer detaches).
    torch.save(torch.randn(3, requires_grad=True), disk.leaf_path(7))
    step = L.load_step(disk, len(leaves), "cpu", threads=3)
    assert step.fallback == 4  # two records, the tensor that needs grad, the empty one
    assert step.leaves[7].requires_grad
    for i in range(len(leaves)):
        a, b = step.leaves[i], disk.leaf(i)
        assert _same(a, b)
        if isinstance(b, torch.Tensor):
            assert a.stride() == b.stride() and a.requires_grad == b.requires_grad
            assert a.untyped_storage().data_ptr() == step.arena.data_ptr()
            if a.numel():
                assert (a.data_ptr() - step.arena.data_ptr()) % L.ALIGN == 0
    assert step.bytes == sum(disk.leaf(i).untyped_storage().nbytes()
                             for i in (2, 3, 4, 5, 6, 9))


def test_loader_leaves_have_their_own_versions(tmp_path):
    leaves = _leaves()
    _, _, _, disk = _write(tmp_path, leaves)
    step = L.load_step(disk, len(leaves), "cpu")
    store = L.ResidentStore(disk, step)
    store.leaf(2).add_(1.0)
    with pytest.raises(StoreMutationError):
        store.leaf(2)
    assert _same(store.leaf(3), leaves[3]) and _same(store.leaf(5), leaves[5])
    assert store.root == disk.root and store.dataset_path(1) == disk.dataset_path(1)


def test_loader_keeps_each_bad_leaf_error_for_its_read(tmp_path):
    leaves = _leaves()
    _, _, _, disk = _write(tmp_path, leaves)
    d = disk.directory
    (d / LEAF_FILE.format(3)).write_bytes(b"\0" * 10)
    torch.save({"x": torch.zeros(2)}, d / LEAF_FILE.format(5))
    (d / LEAF_FILE.format(6)).unlink()
    step = L.load_step(disk, len(leaves) + 1, "cpu")
    store = L.ResidentStore(disk, step)
    for i, err in ((3, LeafReadError), (5, LeafReadError), (6, IndexError), (7, IndexError)):
        with pytest.raises(err):
            disk.leaf(i)
        with pytest.raises(err):
            store.leaf(i)
    assert _same(store.leaf(4), leaves[4])
    with pytest.raises(IndexError):
        store.leaf(8)


def test_loader_brings_captured_operands(tmp_path):
    leaves = _leaves()
    _, _, _, disk = _write(tmp_path, leaves)
    g = torch.Generator().manual_seed(3)
    stacked = torch.randn(2, 6, 5, generator=g).to(torch.bfloat16)
    ops = {4: (stacked[0], torch.randn(5, 3, generator=g)),
           9: (stacked[1], torch.randn(5, 3, generator=g))}
    L.write_operands(disk.directory, ops)
    step = L.load_step(disk, len(leaves), "cpu", operand_ms=[4, 9])
    for m, (a, b) in ops.items():
        assert _same(step.operands[m][0], a) and _same(step.operands[m][1], b)
    with pytest.raises(LeafReadError):
        L.load_step(disk, len(leaves), "cpu", operand_ms=[5])


def test_store_load_rejects_bad_segments_and_short_files(tmp_path):
    p = tmp_path / "x.bin"
    p.write_bytes(bytes(range(256)) * 16)
    table = L._PathTable([p])
    dst = np.zeros(8192, dtype=np.uint8)

    def run(segs):
        s = np.array(segs, dtype=L._SEGMENT)
        return L._lib().pots_store_load(1, table.address, len(s), s.ctypes.data,
                                        dst.ctypes.data, -1, None, 0, 2)

    assert run([(0, 0, 100, 50, 0), (0, 0, 0, 64, 4096)]) == 0
    assert bytes(dst[:50]) == (bytes(range(256)) * 16)[100:150]
    assert bytes(dst[4096:4160]) == bytes(range(64))
    assert run([(0, 0, 0, 64, 100), (0, 0, 0, 64, 0)]) == -4      # not sorted by destination
    assert run([(0, 0, 0, 64, 0), (0, 0, 0, 64, 32)]) == -4       # overlapping
    assert run([(1, 0, 0, 64, 0)]) == -4                          # no such file
    assert run([(0, 0, 4000, 200, 0)]) == -5                      # past the end of the file
    assert "short or failed read" in L._lib().pots_last_error().decode()
