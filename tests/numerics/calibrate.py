"""Calibrate the tolerance constant ``c`` against the vendor fp16 GEMM, then freeze it.

    python -m tests.numerics.calibrate --device cpu --write    # ATen fp16 matmul
    TOKENFORGE_SHAPE_SUITE=full python -m tests.numerics.calibrate --device cuda --write

``c`` is the worst ``max|y_vendor - y_ref| / error_scale`` over every (shape, M, seed) the
numerics tests use plus extra seeds, with ``y_ref`` an fp64 GEMM on the same fp16 inputs,
rounded up to two significant figures (calibrate.py:1-72 in the reference). On the GPU the
vendor GEMM is ``F.linear`` in fp16 on ROCm (hipBLASLt / rocBLAS).
"""

from __future__ import annotations

import argparse
import json
import math
import platform
from pathlib import Path

import numpy as np
import torch

from oracle.pack import dequantize_tf
from tests.numerics import cases
from tests.numerics.shapes import linear_shapes, m_values, suite
from tests.numerics.tolerance import TOLERANCES_PATH, error_scale


def calibrate(device: str) -> dict[str, object]:
    worst = 0.0
    worst_case: tuple[object, ...] = ()
    n_cases = 0
    for shape in linear_shapes():
        for seed in cases.CALIBRATION_SEEDS:
            w16 = dequantize_tf(cases.layer_weights(shape.n, shape.k, seed))
            w64 = w16.astype(np.float64)
            w_dev = torch.from_numpy(w16).to(device)
            for m in m_values():
                x16 = cases.activations(m, shape.k, seed)
                ref = x16.numpy().astype(np.float64) @ w64.T
                y = torch.nn.functional.linear(x16.to(device), w_dev).cpu().numpy().astype(np.float64)
                ratio = float(np.abs(y - ref).max()) / error_scale(x16.numpy(), w16)
                n_cases += 1
                if ratio > worst:
                    worst, worst_case = ratio, (shape.layer, shape.n, shape.k, m, seed)
    exp = math.floor(math.log10(worst))
    c = math.ceil(worst / 10 ** (exp - 1)) * 10 ** (exp - 1)
    return {
        "c": round(c, 6),
        "observed_max": worst,
        "worst_case": list(worst_case),
        "cases": n_cases,
        "suite": suite(),
        "vendor_gemm": "rocm-F.linear-fp16" if device == "cuda" else "aten-cpu-fp16",
        "device_name": torch.cuda.get_device_name() if device == "cuda" else platform.machine(),
        "torch": torch.__version__,
    }


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--device", choices=["cpu", "cuda"], required=True)
    ap.add_argument("--write", action="store_true", help="freeze the result in tolerances.json")
    ap.add_argument("--out", type=str, default=None, help="write the updated tolerances.json here instead")
    args = ap.parse_args()
    result = calibrate(args.device)
    print(json.dumps(result, indent=2), flush=True)
    if args.write or args.out:
        data = json.loads(TOLERANCES_PATH.read_text()) if TOLERANCES_PATH.exists() else {}
        data.setdefault("w4a16", {})[args.device] = result
        target = Path(args.out) if args.out else TOLERANCES_PATH
        target.parent.mkdir(parents=True, exist_ok=True)
        target.write_text(json.dumps(data, indent=2, sort_keys=True) + "\n")


if __name__ == "__main__":
    main()
