"""bench.py's reading of the committed counter summaries (no GPU): each configuration's
``traffic`` comes from its own profile's JSON block, and a configuration with no profile
reports null rather than another's figures."""

from __future__ import annotations

import importlib.util
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("pots_bench", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_traffic_is_read_per_configuration():
    b = _bench()
    kernels = ("chunk_kernel", "row_pass<bf16> (B pass)",
               "row_pass<bf16, weighted> (A pass)", "row_pass<bf16, fp64 squares> (P pass)")
    for k in kernels:
        c4, c5 = b.traffic_from_profile(k, "c4"), b.traffic_from_profile(k, "c5")
        assert c4 is not None and c5 is not None, k
        assert c4 != c5, k
        assert b.traffic_from_profile(k, "c3") is None
    # C4's fused and twin kernels have figures; C5 (k = 16) runs neither
    assert b.traffic_from_profile("chunk_kernel_fused", "c4") is not None
    assert b.traffic_from_profile("twin_pass (A pass of twins)", "c4") is not None
    assert b.traffic_from_profile("chunk_kernel_fused", "c5") is None
    assert b.traffic_from_profile("no_such_kernel", "c4") is None
