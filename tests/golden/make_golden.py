"""Generate ``tests/golden/golden.json``: small committed vectors for the quantized-linear path.

    python -m tests.golden.make_golden

Contents (all produced in this repository; nothing is taken from the reference at run time):

* ``e4m3``: every e4m3fn value, every midpoint, both fp32 neighbours of each midpoint and
  signed zeros (the probe of the reference's test_rmsnorm_fp8.py:89-101), with the codes
  torch's ``.to(torch.float8_e4m3fn)`` produces for them.
* ``repack``: a 64x64 AWQ ``qweight`` (all nibble values present) and its TokenForge
  ``qweight_t``, written out in full, plus the inverse.
* ``gemv_config1``: BASELINE config 1 (M=1, K=N=3584) on seeded inputs: SHA-256 of the
  packed weights and of x, and the fp64 reference output summarized by its first 32 values,
  sum, sum of squares and max.
* ``rmsnorm_fp8_config2``: BASELINE config 2 at T=16 (outlier channels x20): SHA-256 of the
  codes and of the scales of the oracle, and the first row of codes.
"""

from __future__ import annotations

import hashlib
import json
import zlib
from pathlib import Path

import numpy as np
import torch

from oracle import pack as P
from oracle import reference as R

OUT = Path(__file__).with_name("golden.json")


def _sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _seed(*parts: object) -> int:
    return zlib.crc32(repr(parts).encode())


def e4m3_probe() -> np.ndarray:
    values = torch.arange(0, 0x7F, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    mids = (values[1:] + values[:-1]) / 2
    up, down = torch.tensor(1e9), torch.tensor(-1e9)
    probe = torch.cat([values, mids, mids.nextafter(up), mids.nextafter(down)])
    return torch.cat([probe, -probe, torch.tensor([0.0, -0.0])]).numpy()


def config1_inputs() -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """nibbles and zeros uniform [0,15], scales U[1e-3, 1e-2], x ~ N(0,1)."""
    k = n = 3584
    gen = torch.Generator().manual_seed(_seed("config1", 1, n, k, 0))
    intweight = torch.randint(0, 16, (k, n), generator=gen, dtype=torch.int32).numpy()
    zeros = torch.randint(0, 16, (k // 128, n), generator=gen, dtype=torch.int32).numpy()
    scales = (torch.rand((k // 128, n), generator=gen) * 9e-3 + 1e-3).to(torch.float16).numpy()
    x = torch.randn((1, k), generator=gen).to(torch.float16).numpy()
    qweight, qzeros = P.awq_pack(intweight, zeros)
    return qweight, qzeros, scales, x


def config2_inputs(t: int = 16, h: int = 3584) -> tuple[np.ndarray, np.ndarray]:
    chan = torch.randperm(h, generator=torch.Generator().manual_seed(0))[:8]
    gen = torch.Generator().manual_seed(_seed("config2", t, h, 0))
    x = torch.randn((t, h), generator=gen)
    x[:, chan] *= 20.0
    gamma = (1.0 + 0.1 * torch.randn((h,), generator=gen)).to(torch.float16)
    return x.to(torch.float16).numpy(), gamma.numpy()


def main() -> None:
    probe = e4m3_probe()
    codes = torch.from_numpy(probe).to(torch.float8_e4m3fn).view(torch.uint8).numpy()

    rng = np.random.default_rng(1234)
    logical = rng.integers(0, 16, (64, 64), dtype=np.int32)
    logical[0, :16] = np.arange(16)
    awq = P.pack_int4(logical)
    tf = P.repack_awq_to_tf(awq)

    qweight, qzeros, scales, x = config1_inputs()
    w = P.pack_awq(qweight, qzeros, scales, 128)
    y = R.w4a16_reference(x, w)

    xr, gamma = config2_inputs()
    q, s = R.rmsnorm_fp8_reference(xr, gamma, 1e-6)

    doc = {
        "e4m3": {"probe_f32_hex": [f"{int(v):08x}" for v in probe.view(np.uint32)], "codes": codes.tolist()},
        "repack": {
            "k": 64,
            "n": 64,
            "awq_qweight": awq.view(np.uint32).tolist(),
            "tf_qweight_t": tf.view(np.uint32).tolist(),
        },
        "gemv_config1": {
            "m": 1, "n": 3584, "k": 3584, "group_size": 128,
            "sha256_qweight": _sha(qweight), "sha256_qzeros": _sha(qzeros),
            "sha256_scales": _sha(scales), "sha256_x": _sha(x), "sha256_qweight_t": _sha(w.qweight_t),
            "ref_first32": y[0, :32].tolist(), "ref_sum": float(y.sum()), "ref_sumsq": float((y * y).sum()),
            "ref_absmax": float(np.abs(y).max()),
        },
        "rmsnorm_fp8_config2": {
            "t": 16, "h": 3584, "eps": 1e-6,
            "sha256_x": _sha(xr), "sha256_gamma": _sha(gamma),
            "sha256_codes": _sha(q), "sha256_scales": _sha(s),
            "codes_row0_first64": q[0, :64].tolist(),
            "scales": [f"{int(v):08x}" for v in s.view(np.uint32).ravel()],
        },
    }
    OUT.write_text(json.dumps(doc, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
