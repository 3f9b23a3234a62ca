"""The MI355X verifier and commitment engine for pots-2.0's proof-of-training-step hot path.

The module paths mirror the reference's (``verification.commitment``,
``verification.verifier.matmul_check``, ``verification.verifier``,
``verification.computation``), so callers of the reference import the same names. The
arithmetic runs in ``libpots_mi355x.so`` (HIP kernels for gfx950) through
``verification.commitment.native``; there is no CPU fallback.
"""
