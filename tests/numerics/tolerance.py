"""The parity contract of the W4A16 / W4A8 tests: two bounds a kernel's output must meet.

A kernel's fp16 result ``y`` for ``x @ w.T`` (fp16 operands, K = reduction length) is held to

* the derived absolute bound ``c * sqrt(K) * eps_fp16 * max|x| * max|w|`` against the fp64
  product of the same operands: fp32 accumulation makes a length-K dot product's rounding
  error grow like sqrt(K) unit roundoffs of the largest terms, and ``c`` is what the vendor's
  own fp16 GEMM needs on that device class (measured by ``python -m tests.numerics.calibrate``
  and frozen in ``tolerances.json``), so a kernel may be no less accurate than the vendor
  GEMM. This is the reference's measurement contract (tests/numerics/tolerance.py:1-46), with
  one change: the bound holds each output's error above half an fp16 ulp of its fp64 value.
  That half ulp is the rounding of the result to the fp16 output, which even the exact
  product incurs; the reference's form counts it against the bound, so a draw with an output
  of magnitude >= 2 near a rounding midpoint can fail for every fp16 kernel (with K = 384 and
  max|ref| = 2.1 the bound is 9.4e-4 and the half ulp 9.8e-4). The full-size tests use the
  same form.
* the normwise bound ``max|y - ref| / max|ref| <= 1e-2`` against an fp32 dequant-then-matmul,
  the north-star's accuracy target.

Non-finite entries take no part in either bound; their propagation is tested on its own.
Usage: ``contract("cuda").atol(x, w)``, ``contract("cuda").check(y, ref64, ref32, x, w)``.
"""

from __future__ import annotations

import functools
import json
import math
from dataclasses import dataclass
from pathlib import Path

import numpy as np

EPS_FP16 = float(np.finfo(np.float16).eps)  # 2**-10
NORMWISE_MAX = 1e-2
TOLERANCES_PATH = Path(__file__).with_name("tolerances.json")


def _largest_finite(a: np.ndarray) -> float:
    mags = np.abs(np.asarray(a, dtype=np.float64)).ravel()
    mags = mags[np.isfinite(mags)]
    return float(mags.max()) if mags.size else 0.0


def roundoff_scale(x: np.ndarray, w: np.ndarray) -> float:
    """``sqrt(K) * eps_fp16 * max|x| * max|w|`` over finite entries (K = x.shape[-1])."""
    return EPS_FP16 * math.sqrt(x.shape[-1]) * _largest_finite(x) * _largest_finite(w)


def half_ulp_fp16(ref: np.ndarray) -> np.ndarray:
    """Half the fp16 spacing at each |ref| (the largest rounding error of an exact value stored
    as fp16; subnormal spacing below 2**-14)."""
    mag = np.abs(np.asarray(ref, dtype=np.float64))
    binade = np.floor(np.log2(np.maximum(mag, 2.0**-14)))
    return np.exp2(binade - 11)


def relative_max_error(y: np.ndarray, ref: np.ndarray) -> float:
    """``max|y - ref| / max|ref|`` over the entries where ``ref`` is finite (the absolute
    error when ``ref`` is all zero)."""
    r = np.asarray(ref, dtype=np.float64)
    finite = np.isfinite(r)
    if not finite.any():
        return 0.0
    err = float(np.max(np.abs(np.asarray(y, dtype=np.float64)[finite] - r[finite])))
    peak = float(np.max(np.abs(r[finite])))
    return err / peak if peak > 0 else err


@dataclass(frozen=True)
class Outcome:
    """Measured errors of one output next to the bounds they are held to."""

    abs_err: float
    atol: float
    normwise: float

    @property
    def ok(self) -> bool:
        return self.abs_err <= self.atol and self.normwise <= NORMWISE_MAX

    def __str__(self) -> str:
        return (f"abs above half an fp16 ulp {self.abs_err:.3e} (bound {self.atol:.3e}), "
                f"normwise {self.normwise:.3e} (bound {NORMWISE_MAX})")


@dataclass(frozen=True)
class Contract:
    """The bounds of one device class ("cpu" or "cuda"), with its frozen constant ``c``."""

    device: str
    c: float

    def atol(self, x: np.ndarray, w: np.ndarray) -> float:
        return self.c * roundoff_scale(x, w)

    def check(self, y: np.ndarray, ref64: np.ndarray, ref32: np.ndarray, x: np.ndarray, w: np.ndarray) -> Outcome:
        """``y`` against the fp64 product ``ref64`` (absolute bound on the error above half an
        fp16 ulp of each output, finite entries) and the fp32 dequant-then-matmul ``ref32``
        (normwise bound)."""
        y64 = np.asarray(y, dtype=np.float64)
        r64 = np.asarray(ref64, dtype=np.float64)
        finite = np.isfinite(r64)
        excess = np.abs(y64[finite] - r64[finite]) - half_ulp_fp16(r64[finite])
        abs_err = float(max(0.0, np.max(excess))) if finite.any() else 0.0
        return Outcome(abs_err, self.atol(x, w), relative_max_error(y64, ref32))


@functools.cache
def _frozen_table(path: Path) -> dict:  # type: ignore[type-arg]
    return json.loads(path.read_text()).get("w4a16", {})


def contract(device: str, path: Path = TOLERANCES_PATH) -> Contract:
    """The contract frozen in ``tolerances.json`` for ``device``; LookupError if it was never
    calibrated there."""
    table = _frozen_table(path)
    if device not in table:
        raise LookupError(
            f"no calibrated tolerance for device '{device}'; run "
            f"`python -m tests.numerics.calibrate --device {device} --write` once and commit it"
        )
    return Contract(device, float(table[device]["c"]))
