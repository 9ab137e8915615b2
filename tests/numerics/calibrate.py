"""Measure the tolerance constant ``c`` on the vendor fp16 GEMM and freeze it.

    python -m tests.numerics.calibrate --device cpu --write    # ATen fp16 matmul
    TOKENFORGE_SHAPE_SUITE=full python -m tests.numerics.calibrate --device cuda --write

For every (shape, M, seed) the numerics tests use, plus extra seeds, the vendor GEMM's
error against an fp64 product of the same fp16 operands is divided by
``tolerance.error_scale``; ``c`` is the largest such ratio rounded up to two significant
digits (the reference's calibration procedure, tests/numerics/calibrate.py:1-72). On the GPU
the vendor GEMM is ``F.linear`` in fp16 on ROCm (hipBLASLt / rocBLAS).
"""

from __future__ import annotations

import argparse
import json
import math
import platform
from collections.abc import Iterator
from pathlib import Path

import numpy as np
import torch

from oracle.pack import dequantize_tf
from tests.numerics import cases
from tests.numerics.shapes import linear_shapes, m_values, suite
from tests.numerics.tolerance import TOLERANCES_PATH, error_scale


def _vendor_ratios(device: str) -> Iterator[tuple[float, tuple[object, ...]]]:
    """(error / error_scale, case id) of the vendor fp16 GEMM on every calibration case."""
    for shape in linear_shapes():
        for seed in cases.CALIBRATION_SEEDS:
            w16 = dequantize_tf(cases.layer_weights(shape.n, shape.k, seed))
            w_on_device = torch.from_numpy(w16).to(device)
            for m in m_values():
                x16 = cases.activations(m, shape.k, seed)
                exact = x16.numpy().astype(np.float64) @ w16.astype(np.float64).T
                got = torch.nn.functional.linear(x16.to(device), w_on_device).cpu().numpy()
                err = float(np.abs(got.astype(np.float64) - exact).max())
                yield err / error_scale(x16.numpy(), w16), (shape.layer, shape.n, shape.k, m, seed)


def round_up_2sig(v: float) -> float:
    """Smallest two-significant-digit number >= v (v > 0)."""
    step = 10.0 ** (math.floor(math.log10(v)) - 1)
    return round(math.ceil(v / step) * step, 6)


def calibrate(device: str) -> dict[str, object]:
    ratios = list(_vendor_ratios(device))
    worst, worst_case = max(ratios, key=lambda r: r[0])
    return {
        "c": round_up_2sig(worst),
        "observed_max": worst,
        "worst_case": list(worst_case),
        "cases": len(ratios),
        "suite": suite(),
        "vendor_gemm": "rocm-F.linear-fp16" if device == "cuda" else "aten-cpu-fp16",
        "device_name": torch.cuda.get_device_name() if device == "cuda" else platform.machine(),
        "torch": torch.__version__,
    }


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--device", choices=["cpu", "cuda"], required=True)
    ap.add_argument("--write", action="store_true", help="freeze the result in tolerances.json")
    ap.add_argument("--out", type=str, default=None, help="write the updated tolerances.json here instead")
    args = ap.parse_args()
    entry = calibrate(args.device)
    print(json.dumps(entry, indent=2), flush=True)
    if not (args.write or args.out):
        return
    table = json.loads(TOLERANCES_PATH.read_text()) if TOLERANCES_PATH.exists() else {}
    table.setdefault("w4a16", {})[args.device] = entry
    target = Path(args.out) if args.out else TOLERANCES_PATH
    target.parent.mkdir(parents=True, exist_ok=True)
    target.write_text(json.dumps(table, indent=2, sort_keys=True) + "\n")


if __name__ == "__main__":
    main()
