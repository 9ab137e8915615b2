"""Derived numerical tolerance for the W4A16 kernels (tolerance.py:1-46 in the reference).

With fp32 accumulation the error grows like sqrt(K), so

    atol = c * sqrt(K) * eps_fp16 * max|x| * max|w|

``c`` is calibrated once per device class against the vendor fp16 GEMM (hipBLASLt/rocBLAS
through ``F.linear`` on the GPU, ATen's fp16 matmul on CPU) by
``python -m tests.numerics.calibrate`` and frozen in ``tolerances.json``. A kernel that
needs a looser constant than the vendor GEMM fails.

The second check, :func:`normwise`, is the north-star bound: ``max|y - ref| / max|ref|``
against an fp32 dequant-then-matmul must stay at or below 1e-2.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np

EPS_FP16 = float(np.finfo(np.float16).eps)  # 2**-10
TOLERANCES_PATH = Path(__file__).with_name("tolerances.json")
NORMWISE_MAX = 1e-2


def error_scale(x: np.ndarray, w: np.ndarray) -> float:
    """``sqrt(K) * eps_fp16 * max|x| * max|w|`` over finite entries."""
    k = x.shape[-1]
    xf = np.asarray(x, dtype=np.float64)
    wf = np.asarray(w, dtype=np.float64)
    finite = np.isfinite(xf)
    xmax = float(np.abs(xf[finite]).max()) if finite.any() else 0.0
    wmax = float(np.abs(wf).max()) if wf.size else 0.0
    return math.sqrt(k) * EPS_FP16 * xmax * wmax


def load_constant(device_type: str) -> float:
    data = json.loads(TOLERANCES_PATH.read_text())
    entry = data["w4a16"].get(device_type)
    if entry is None:
        raise LookupError(
            f"no calibrated tolerance for device '{device_type}'; run "
            f"`python -m tests.numerics.calibrate --device {device_type} --write` once and commit it"
        )
    return float(entry["c"])


def atol(x: np.ndarray, w: np.ndarray, device_type: str) -> float:
    return load_constant(device_type) * error_scale(x, w)


def normwise(y: np.ndarray, ref: np.ndarray) -> float:
    """``max|y - ref| / max|ref|`` over finite reference entries."""
    y64 = np.asarray(y, dtype=np.float64)
    r64 = np.asarray(ref, dtype=np.float64)
    finite = np.isfinite(r64)
    denom = float(np.abs(r64[finite]).max()) if finite.any() else 0.0
    err = float(np.abs(y64[finite] - r64[finite]).max()) if finite.any() else 0.0
    return err / denom if denom > 0 else err
