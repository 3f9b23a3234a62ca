"""Write tests/golden/leaf_digests.json: tensor-leaf digests at the reference's edge shapes.

Each digest is computed by the C oracle (incremental BLAKE3, chaining-value stack) and, for
leaves up to 1 MiB, recomputed by the independent pure-Python BLAKE3 (recursive split); the
script refuses to write a digest the two disagree on. Run from the repository root:

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT / "oracle"), str(ROOT / "tests" / "golden")]

import blake3_tree  # noqa: E402
import oracle  # noqa: E402
from payloads import DTYPES, SHAPES, payload  # noqa: E402


def main() -> None:
    out = []
    for di, (dname, dtype) in enumerate(DTYPES.items()):
        for si, shape in enumerate(SHAPES):
            seed = 1000 * di + si
            t = payload(shape, dtype, seed)
            for tag in (oracle.TAG_WEIGHT, oracle.TAG_PRODUCT):
                hdr = oracle.tensor_leaf_header(tag, t)
                msg = b"\x00" + hdr + oracle.payload_bytes(t)
                d = oracle.blake3(msg)
                if len(msg) <= 1 << 20:
                    assert blake3_tree.blake3(msg) == d, (dname, shape)
                out.append({"dtype": dname, "shape": list(shape), "seed": seed, "tag": tag,
                            "digest": d.hex()})
    path = Path(__file__).with_name("leaf_digests.json")
    path.write_text(json.dumps(out, indent=0) + "\n")
    print(f"wrote {len(out)} digests to {path}")


if __name__ == "__main__":
    main()
