"""Build libpots_mi355x.so for gfx950 from csrc/*.hip with hipcc, in place.

    python pots-2.0_amd/build.py

The library lands next to this file, so it travels with the source tree to the GPU host.
Every HIP source is compiled with packed FP32 instructions switched off
(``-Xclang -target-feature -Xclang -packed-fp32-ops``) and without fast-math, so the fp64
verdict arithmetic keeps IEEE semantics. Matrix-core instructions take their accumulators in
ordinary VGPRs (``-amdgpu-mfma-vgpr-form``): the row and twin passes then keep them there
instead of copying them between VGPRs and AGPRs around every MFMA (the twin pass's loop went
from 142 to 111 VALU instructions per 16-row stage, and every row pass lost its copies).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "csrc"
LIB = HERE / "libpots_mi355x.so"
ARCH = os.environ.get("POTS_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def flags() -> list[str]:
    return ["-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-ffp-contract=off", "-fno-fast-math", "-mllvm", "-amdgpu-mfma-vgpr-form=1",
            "-Wall", "-Wno-unused-function",
            f"-I{HERE.parent / 'include'}"]


def build(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip into object files, then link the shared library."""
    sources = sorted(SRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {SRC}")
    obj_dir = HERE / "_build"
    obj_dir.mkdir(exist_ok=True)
    cc = hipcc()
    objs = []
    procs = []
    for src in sources:
        obj = obj_dir / (src.stem + ".o")
        objs.append(obj)
        cmd = [cc, *flags(), "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                            stderr=subprocess.STDOUT, text=True)))
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        if p.returncode != 0:
            failed.append(f"{src.name}:\n{out}")
        elif verbose and out.strip():
            print(out, flush=True)
    if failed:
        raise RuntimeError("hipcc failed:\n" + "\n".join(failed))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
