"""Measure the constant ``c`` of the derived bound on the vendor fp16 GEMM, and freeze it.

    python -m tests.numerics.calibrate --device cpu --write    # ATen fp16 matmul
    TOKENFORGE_SHAPE_SUITE=full python -m tests.numerics.calibrate --device cuda --write
    python -m tests.numerics.calibrate --device cuda --baseline-sizes --write

Every (shape, M) of the active shape suite is run on the numerics tests' inputs for each
calibration seed. Each run's error (vendor fp16 ``F.linear`` against the fp64 product of the
same fp16 operands) is expressed in units of ``tolerance.roundoff_scale``; ``c`` is the
largest such ratio rounded up to two significant digits, so the vendor GEMM itself just meets
the bound (the reference's procedure, tests/numerics/calibrate.py:1-72). On ROCm the vendor
GEMM is hipBLASLt / rocBLAS.
"""

from __future__ import annotations

import argparse
import json
import math
import platform
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from oracle.pack import dequantize_tf
from tests.numerics import cases, shapes
from tests.numerics.tolerance import EPS_FP16, TOLERANCES_PATH, roundoff_scale


@dataclass(frozen=True)
class Sample:
    layer: str
    n: int
    k: int
    m: int
    seed: int
    ratio: float  # vendor error / roundoff_scale


def measure(device: str, suite: shapes.ShapeSuite) -> list[Sample]:
    samples = []
    for shape in suite.shapes:
        for seed in cases.CALIBRATION_SEEDS:
            w16 = dequantize_tf(cases.layer_weights(shape.n, shape.k, seed))
            w_dev = torch.from_numpy(w16).to(device)
            w64 = w16.astype(np.float64)
            for m in suite.m_values:
                x16 = cases.activations(m, shape.k, seed)
                vendor = torch.nn.functional.linear(x16.to(device), w_dev).cpu().numpy().astype(np.float64)
                err = float(np.abs(vendor - x16.numpy().astype(np.float64) @ w64.T).max())
                samples.append(Sample(shape.layer, shape.n, shape.k, m, seed, err / roundoff_scale(x16.numpy(), w16)))
    return samples


def two_digits_up(v: float) -> float:
    """The smallest number with two significant digits that is >= v (v > 0)."""
    unit = 10.0 ** (math.floor(math.log10(v)) - 1)
    return round(math.ceil(v / unit) * unit, 6)


def table_entry(device: str, suite: shapes.ShapeSuite, samples: list[Sample]) -> dict[str, object]:
    worst = max(samples, key=lambda s: s.ratio)
    return {
        "c": two_digits_up(worst.ratio),
        "observed_max": worst.ratio,
        "worst_case": [worst.layer, worst.n, worst.k, worst.m, worst.seed],
        "cases": len(samples),
        "suite": suite.name,
        "vendor_gemm": "rocm-F.linear-fp16" if device == "cuda" else "aten-cpu-fp16",
        "device_name": torch.cuda.get_device_name() if device == "cuda" else platform.machine(),
        "torch": torch.__version__,
    }


def freeze(device: str, entry: dict[str, object], target: Path) -> None:
    """Merge ``entry`` into the tolerances table at ``target`` (read from the committed table)."""
    table = json.loads(TOLERANCES_PATH.read_text()) if TOLERANCES_PATH.exists() else {}
    table.setdefault("w4a16", {})[device] = entry
    target.parent.mkdir(parents=True, exist_ok=True)
    target.write_text(json.dumps(table, indent=2, sort_keys=True) + "\n")


BASELINE_CASES = (("o_proj", 3584, 3584, (1,)),
                  ("gate_up", 37888, 3584, (16, 32, 64, 128, 256, 1024, 4096)),
                  ("down", 3584, 18944, (16, 32, 64, 128, 256, 1024, 4096)))


def measure_baseline_sizes(device: str) -> dict[str, object]:
    """The vendor fp16 GEMM on BASELINE configs 1 and 4 at full size (weights from
    ``cases.baseline_layer``, x ~ N(0, 1) with 1% of the rows scaled by 10 at M >= 16), against
    the fp32 product on the device, in units of the derived bound's roundoff scale: the plain
    error, and the error above half an fp16 ulp of each output (the full-size tests' form).
    At these magnitudes the final fp16 rounding of an output alone can exceed c times the
    roundoff scale, which is what the half ulp accounts for."""
    from oracle.pack import pack_awq

    rows = []
    for layer, n, k, ms in BASELINE_CASES:
        qweight, qzeros, scales = cases.baseline_layer(n, k, 0)
        w16 = dequantize_tf(pack_awq(qweight, qzeros, scales, cases.GROUP_SIZE))
        w_dev = torch.from_numpy(w16).to(device)
        wt32 = w_dev.float().t().contiguous()
        wmax = float(np.abs(w16.astype(np.float32)).max())
        for m in ms:
            gen = torch.Generator().manual_seed(m)
            x = torch.randn((m, k), generator=gen)
            if m >= 16:
                x[torch.randperm(m, generator=gen)[: math.ceil(0.01 * m)]] *= 10
            x = x.to(torch.float16).to(device)
            ref = x.float() @ wt32
            vendor = torch.nn.functional.linear(x, w_dev).float()
            scale = EPS_FP16 * math.sqrt(k) * float(x.float().abs().max()) * wmax
            half_ulp = torch.from_numpy(np.spacing(np.abs(ref.cpu().numpy()).astype(np.float16)).astype(np.float32)).to(device) / 2
            err = (vendor - ref).abs()
            rows.append({"layer": layer, "n": n, "k": k, "m": m, "plain": float(err.max()) / scale,
                         "above_half_ulp": float((err - half_ulp).max()) / scale})
    return {"cases": rows, "max_plain": max(r["plain"] for r in rows),
            "max_above_half_ulp": max(r["above_half_ulp"] for r in rows),
            "vendor_gemm": "rocm-F.linear-fp16" if device == "cuda" else "aten-cpu-fp16",
            "torch": torch.__version__}


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--device", choices=["cpu", "cuda"], required=True)
    ap.add_argument("--write", action="store_true", help="freeze the result in tolerances.json")
    ap.add_argument("--out", type=Path, default=None, help="write the updated table here instead")
    ap.add_argument("--baseline-sizes", action="store_true",
                    help="measure the vendor GEMM at BASELINE configs 1 and 4 (full size) instead")
    args = ap.parse_args()
    if args.baseline_sizes:
        entry = measure_baseline_sizes(args.device)
        print(json.dumps(entry, indent=2), flush=True)
        if args.write or args.out:
            target = args.out or TOLERANCES_PATH
            table = json.loads(TOLERANCES_PATH.read_text()) if TOLERANCES_PATH.exists() else {}
            table.setdefault("w4a16_baseline_sizes", {})[args.device] = entry
            target.parent.mkdir(parents=True, exist_ok=True)
            target.write_text(json.dumps(table, indent=2, sort_keys=True) + "\n")
        return
    suite = shapes.active()
    entry = table_entry(args.device, suite, measure(args.device, suite))
    print(json.dumps(entry, indent=2), flush=True)
    if args.write or args.out:
        freeze(args.device, entry, args.out or TOLERANCES_PATH)


if __name__ == "__main__":
    main()
