"""Tolerances of the W4A16 parity tests.

Two bounds, both against references computed from the same fp16 inputs:

* **Derived absolute bound** (the reference's measurement contract, tests/numerics/
  tolerance.py:1-46): with fp32 accumulation the rounding error of a length-K dot product
  grows like sqrt(K) times the unit roundoff times the largest operands, so a kernel's error
  against the fp64 product is bounded by ``c * sqrt(K) * eps_fp16 * max|x| * max|w|``. The
  constant ``c`` is measured once per device class on the vendor fp16 GEMM
  (``python -m tests.numerics.calibrate``) and frozen in ``tolerances.json``: a kernel that
  needs a looser constant than the vendor GEMM fails.
* **Normwise bound** (the north-star contract): ``max|y - ref| / max|ref| <= 1e-2`` against
  an fp32 dequant-then-matmul.

Non-finite entries are left out of both (they are checked for propagation separately).
"""

from __future__ import annotations

import json
import math
from dataclasses import dataclass
from pathlib import Path

import numpy as np

EPS_FP16 = float(np.finfo(np.float16).eps)  # 2**-10
TOLERANCES_PATH = Path(__file__).with_name("tolerances.json")
NORMWISE_MAX = 1e-2


def _finite_absmax(a: np.ndarray) -> float:
    v = np.abs(np.asarray(a, dtype=np.float64))
    v = v[np.isfinite(v)]
    return float(v.max()) if v.size else 0.0


def error_scale(x: np.ndarray, w: np.ndarray) -> float:
    """``sqrt(K) * eps_fp16 * max|x| * max|w|`` (K = x's last dimension)."""
    return math.sqrt(x.shape[-1]) * EPS_FP16 * _finite_absmax(x) * _finite_absmax(w)


@dataclass(frozen=True)
class Calibration:
    """One frozen entry of ``tolerances.json``: the constant and where it came from."""

    device_type: str
    c: float

    @classmethod
    def load(cls, device_type: str, path: Path = TOLERANCES_PATH) -> Calibration:
        table = json.loads(path.read_text()).get("w4a16", {})
        if device_type not in table:
            raise LookupError(
                f"no calibrated tolerance for device '{device_type}'; run "
                f"`python -m tests.numerics.calibrate --device {device_type} --write` once and commit it"
            )
        return cls(device_type, float(table[device_type]["c"]))

    def bound(self, x: np.ndarray, w: np.ndarray) -> float:
        return self.c * error_scale(x, w)


def load_constant(device_type: str) -> float:
    return Calibration.load(device_type).c


def atol(x: np.ndarray, w: np.ndarray, device_type: str) -> float:
    """Derived absolute bound for ``x @ w.T`` on ``device_type`` ("cuda" or "cpu")."""
    return Calibration.load(device_type).bound(x, w)


def normwise(y: np.ndarray, ref: np.ndarray) -> float:
    """``max|y - ref| / max|ref|`` over the entries where ``ref`` is finite."""
    r = np.asarray(ref, dtype=np.float64)
    keep = np.isfinite(r)
    if not keep.any():
        return 0.0
    diff = float(np.abs(np.asarray(y, dtype=np.float64)[keep] - r[keep]).max())
    scale = float(np.abs(r[keep]).max())
    return diff / scale if scale > 0 else diff
