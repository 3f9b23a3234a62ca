"""The tolerances of check 5 (reference: verification/verifier/bands.py:41-157).

``tau`` is the one dimensionless ``τ`` of test 2; ``kappa_max`` the default cancellation
ceiling of test 1, overridden per product class by ``kappa_classes``. Provisional bands are
``τ = 8``, ``κ_max = 1e4``. A band file is JSON; its ``source`` identifies the file.
"""

from __future__ import annotations

import hashlib
import json
import math
import re
from collections.abc import Mapping
from dataclasses import dataclass, field
from pathlib import Path
from types import MappingProxyType
from typing import Any

from verification.verifier.matmul_check.sizing import Z

TAU_W0 = 4.0
KAPPA_PROVISIONAL = 1e4
BAND_FILE_VERSION = 1


def _frozen(m: Mapping[str, float]) -> Mapping[str, float]:
    return MappingProxyType({str(k): float(v) for k, v in dict(m).items()})


@dataclass(frozen=True)
class Bands:
    tau: float
    kappa_max: float
    tau_w: float = TAU_W0
    kappa_classes: Mapping[str, float] = field(default_factory=dict)
    tau_w_tensors: Mapping[str, float] = field(default_factory=dict)
    source: str = "provisional"
    stats: Mapping[str, Any] = field(default_factory=dict, compare=False)

    def __post_init__(self) -> None:
        object.__setattr__(self, "kappa_classes", _frozen(self.kappa_classes))
        object.__setattr__(self, "tau_w_tensors", _frozen(self.tau_w_tensors))
        object.__setattr__(self, "stats", MappingProxyType(dict(self.stats)))
        if not (math.isfinite(self.tau) and self.tau > 0):
            raise ValueError(f"tau must be positive and finite, got {self.tau}")
        for name, v in [("kappa_max", self.kappa_max), *self.kappa_classes.items()]:
            if not (math.isfinite(v) and v >= 1):
                raise ValueError(f"κ_max {name} = {v}: a cancellation factor is ≥ 1")
        for name, v in [("tau_w", self.tau_w), *self.tau_w_tensors.items()]:
            if not (math.isfinite(v) and v >= TAU_W0):
                raise ValueError(f"τ_W {name} = {v} is below the analytic floor {TAU_W0}")

    @classmethod
    def provisional(cls) -> Bands:
        """``τ = Z·1 = 8``, ``κ_max = 1e4``, ``τ_W = 4``."""
        return cls(tau=Z * 1.0, kappa_max=KAPPA_PROVISIONAL, tau_w=TAU_W0)

    def kappa_for(self, cls_key: str) -> float:
        return self.kappa_classes.get(cls_key, self.kappa_max)

    def tau_w_for(self, weight: str) -> float:
        return self.tau_w_tensors.get(weight, self.tau_w)

    def to_dict(self) -> dict[str, Any]:
        return {"version": BAND_FILE_VERSION, "tau": self.tau,
                "kappa_max": {"default": self.kappa_max, "classes": dict(self.kappa_classes)},
                "tau_w": {"default": self.tau_w, "tensors": dict(self.tau_w_tensors)},
                "stats": dict(self.stats)}

    def to_json(self) -> bytes:
        return json.dumps(self.to_dict(), sort_keys=True, indent=1).encode()

    @classmethod
    def from_dict(cls, d: Mapping[str, Any], *, source: str) -> Bands:
        if d.get("version") != BAND_FILE_VERSION:
            raise ValueError(f"band file version {d.get('version')!r}, "
                             f"expected {BAND_FILE_VERSION}")
        return cls(tau=float(d["tau"]), kappa_max=float(d["kappa_max"]["default"]),
                   kappa_classes=d["kappa_max"].get("classes", {}),
                   tau_w=float(d["tau_w"]["default"]),
                   tau_w_tensors=d["tau_w"].get("tensors", {}), source=source,
                   stats=d.get("stats", {}))

    @classmethod
    def from_json(cls, b: bytes) -> Bands:
        """Bands from band-file bytes. The reference names the file by its BLAKE3 hex; this
        build names it by its SHA-256 hex, prefixed ``sha256:`` so the two never collide."""
        return cls.from_dict(json.loads(b), source="sha256:" + hashlib.sha256(b).hexdigest())

    @classmethod
    def from_file(cls, path: str | Path) -> Bands:
        return cls.from_json(Path(path).read_bytes())


_DIGITS = re.compile(r"\d+")


def product_class(c: Any, spec: Any) -> str:
    """A product's calibration class: ``C.product_class(spec)`` when declared, else its kind
    and role with digit runs replaced by ``*``."""
    own = getattr(c, "product_class", None)
    if callable(own):
        return str(own(spec))
    role = spec.weight if spec.weight is not None else spec.name
    return f"{spec.kind.value}:{_DIGITS.sub('*', role)}"
