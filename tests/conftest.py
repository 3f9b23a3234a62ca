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


def started_verifier(c, leaves, *, k, n_steps=1, **kw):
    """A started ``Verifier`` (the reference's constructor) for a run whose first step is
    ``leaves``: ``W_0`` is that step's ``W_t``, ``D`` its records in batch order (so ``π(t)``
    is ``0..n_s−1``), ``h_D`` their root; provisional bands unless given; captured operands
    trusted when the computation serves them."""
    from verification.commitment.leaves import leaf_hashes_of
    from verification.commitment.merkle import merkle_root
    from verification.verifier.bands import Bands
    from verification.verifier.driver import Verifier
    records = [leaves[c.record_index(i)] for i in range(c.n_s)]
    h_D = merkle_root(leaf_hashes_of(c, ((0, r) for r in records)))
    w0 = {name: leaves[c.w_t_index(name)].detach().clone() for name in c.weight_names}
    kw.setdefault("bands", None if kw.get("calibrate") else Bands.provisional())
    kw.setdefault("allow_provisional", True)
    captured = getattr(getattr(c, "_operands", None), "prover_supplied", False)
    kw.setdefault("trust_prover_operands", bool(captured))
    v = Verifier(c, h_D=h_D, n_records=c.n_s, k=k, n_steps=n_steps, seed=0, w0=w0,
                 schedule=lambda t: list(range(c.n_s)), **kw)
    assert v.start_run(records) is None
    return v
