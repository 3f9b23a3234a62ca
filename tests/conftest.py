"""Test configuration: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs the oracle against the reference's known answers, the host-side logic,
and the C ABI's exports; ``-m gpu`` runs the parity tests of the HIP kernels against the
oracle on a GPU.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "pots-2.0_amd", ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built library")


@pytest.fixture(scope="session")
def lib():
    """The product library on the GPU; fails loudly if it is missing."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    from verification.commitment import native
    return native.get()
