"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.

The store reader parses the prover's torch.save files, which are untrusted input, and the
plan builders turn the verifier's tables into device metadata. Both are built for the host
alone by ``pots-2.0_amd/csrc/host_check/Makefile`` (every HIP source compiled host-only with
``-fsanitize=address,undefined``, a host model in place of the HIP runtime) into the
``host_check`` driver, which the tests run as a child process with the sanitizers set to stop
at their first finding:

- the scan and the host-mode load over the damaged-file corpus of test_store_host.py (bytes
  changed in the archive and in the pickle of two tensors, 300 files each) and the files the
  scan must leave to torch.load; every file's outcome must equal the production library's,
  and every storage the scan takes must load to the file's own bytes;
- 300 randomized Freivalds plans (shapes, strides, dtypes, biases, twins, k, guard) and the
  leaf plans over their products, fused and not, with the refusals the generator expects.
"""

from __future__ import annotations

import os
import random
import shutil
import subprocess
import zipfile
from pathlib import Path

import pytest
import torch

from verification.transcript import loader as L

HERE = Path(__file__).resolve().parent
CHECK = HERE.parent / "pots-2.0_amd" / "csrc" / "host_check"
ENV = {"ASAN_OPTIONS": "halt_on_error=1:abort_on_error=0:detect_leaks=1",
       "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}


@pytest.fixture(scope="module")
def driver() -> Path:
    if shutil.which("make") is None or not Path("/opt/rocm/bin/hipcc").exists():
        pytest.skip("needs make and hipcc")
    r = subprocess.run(["make", "-C", str(CHECK), f"-j{min(8, os.cpu_count() or 1)}"],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    return CHECK / "_build" / "host_check"


def _run(driver: Path, *args: str) -> str:
    r = subprocess.run([str(driver), *args], capture_output=True, text=True, timeout=600,
                       env={**os.environ, **ENV})
    assert r.returncode == 0 and "Sanitizer" not in r.stderr and \
        "runtime error" not in r.stderr, r.stderr[-4000:]
    return r.stdout


def _fnv1a(b: bytes) -> int:
    h = 1469598103934665603
    for x in b:
        h = ((h ^ x) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h


def _damaged(tmp: Path, region: str, tensor: str) -> list[Path]:
    """test_store_host.py's damaged-file corpus for one (region, tensor)."""
    from test_store_host import _record_span
    t = (torch.arange(60, dtype=torch.float32).reshape(6, 10) if tensor == "f32" else
         torch.randn(3, 4, 50, generator=torch.Generator().manual_seed(0))
         .to(torch.bfloat16).permute(2, 0, 1))
    src = tmp / f"{region}_{tensor}.pt"
    torch.save(t, src)
    raw = src.read_bytes()
    with zipfile.ZipFile(src) as zf:
        data_lo, data_hi = _record_span(raw, next(i for i in zf.infolist()
                                                  if "/data/" in i.filename))
        pk_lo, pk_hi = _record_span(raw, next(i for i in zf.infolist()
                                              if i.filename.endswith("/data.pkl")))
    rng = random.Random({"archive": 7, "pickle": 11}[region] + 100 * (tensor == "f32"))
    out = [src]
    for k in range(300):
        b = bytearray(raw)
        for _ in range(rng.choice((1, 1, 2, 3, 5))):
            while True:
                pos = rng.randrange(pk_lo, pk_hi) if region == "pickle" else \
                    rng.randrange(len(b))
                if not data_lo <= pos < data_hi:
                    break
            b[pos] = rng.randrange(256)
        p = tmp / f"{region}_{tensor}_{k}.pt"
        p.write_bytes(bytes(b))
        out.append(p)
    return out


def _others(tmp: Path) -> list[Path]:
    """Files the scan must leave to torch.load, and some it takes."""
    objs = {"record": {"ids": torch.zeros(3, dtype=torch.int32)},
            "grad": torch.randn(3, requires_grad=True), "empty": torch.zeros(0, 4),
            "pair": (torch.zeros(2), torch.ones(2)), "int": 7,
            "scalar": torch.tensor(2.5), "view": torch.arange(40.0).reshape(5, 8)[1:3, 2:6],
            "big": torch.randn(300, 700), "bool": torch.rand(9) > 0.5}
    out = []
    for name, obj in objs.items():
        torch.save(obj, tmp / f"o_{name}.pt")
        out.append(tmp / f"o_{name}.pt")
    (tmp / "o_junk.pt").write_bytes(b"not a torch file")
    (tmp / "o_short.pt").write_bytes(b"PK")
    (tmp / "o_empty.pt").write_bytes(b"")
    return out + [tmp / "o_junk.pt", tmp / "o_short.pt", tmp / "o_empty.pt",
                  tmp / "o_missing.pt"]


@pytest.mark.filterwarnings("ignore:Detected pickle protocol")
def test_store_reader_is_clean_on_damaged_and_foreign_files(driver, tmp_path):
    paths = _others(tmp_path)
    for region in ("archive", "pickle"):
        for tensor in ("f32", "bf16_permuted"):
            paths += _damaged(tmp_path, region, tensor)
    lines = _run(driver, "scan", *map(str, paths)).splitlines()
    assert len(lines) == len(paths)
    info = L.scan_files(paths, threads=4)
    taken = 0
    for p, r, line in zip(paths, info, lines):
        got = line.split()
        assert int(got[0]) == int(r["status"]), (p, line)
        if int(r["status"]) != L.STORE_OK:
            continue
        taken += 1
        nd = int(r["ndim"])
        want = [int(r["ndim"]), int(r["dtype"]), int(r["data_offset"]),
                int(r["storage_bytes"]), int(r["storage_offset"]),
                *r["size"][:nd].tolist()]
        assert [int(x) for x in got[1:6 + nd]] == want, (p, line)
        assert got[6 + nd] == "/"
        assert [int(x) for x in got[7 + nd:7 + 2 * nd]] == r["stride"][:nd].tolist()
        raw = p.read_bytes()
        lo = int(r["data_offset"])
        data = raw[lo:lo + int(r["storage_bytes"])]
        assert int(got[-1], 16) == _fnv1a(data), p
    assert 10 < taken < len(paths)


def test_plan_builders_are_clean_under_sanitizers(driver):
    out = _run(driver, "plans", "11", "300")
    assert out.startswith("plans ok: 300")
    twins, fused = (int(x) for x in out.split("(")[1].split()[0:4:2])
    assert twins > 0 and fused > 0  # the generator reached the twin pass and the fusion


def test_sanitizers_are_live_in_the_driver(driver):
    """The driver is instrumented: the ASan and UBSan runtimes are linked into it."""
    syms = subprocess.run(["nm", str(driver)], capture_output=True, text=True).stdout
    assert "__asan_init" in syms and "__ubsan_handle" in syms
