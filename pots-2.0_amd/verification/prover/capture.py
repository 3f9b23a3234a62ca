"""The prover's matmul capture (reference: verification/prover/capture.py:1-602).

The recorder itself lives in :mod:`verification.computation.recording`, beside the other
pieces the prover and the verifier's replay share; this module is the prover's name for it.
"""

from verification.computation.recording import (PHASES, BiasedMatmulError, CaptureError,
                                                CopyRecord, MatmulCapture, MatmulRecord,
                                                MutatedCaptureError, OperandInfo, PhaseError,
                                                UnsupportedMatmulError)

__all__ = ["PHASES", "CaptureError", "UnsupportedMatmulError", "BiasedMatmulError",
           "PhaseError", "MutatedCaptureError", "OperandInfo", "MatmulRecord", "CopyRecord",
           "MatmulCapture"]
