"""The RMSNorm+FP8 kernel's per-row divisions (tokenforge_amd/csrc/norm_row.h): amax / 448
and the mean sum / h are computed as fp32(fp64(value) * fp64(1 / divisor)). Both equal the IEEE
fp32 quotients: every positive finite fp16 amax, and sampled fp32 sums (exact multiples of h,
and values across fp16's squared range) with every row width h up to 32768. The dynamic-scale
quotient y / s is checked exhaustively on the GPU in tests/gpu/test_norm_quotient.py.
"""

from __future__ import annotations

import numpy as np


def _positive_finite_fp16() -> np.ndarray:
    return np.arange(1, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)


def test_absmax_over_448_as_reciprocal_product() -> None:
    amax = _positive_finite_fp16()
    ieee = amax / np.float32(448.0)
    product = (amax.astype(np.float64) * (1.0 / 448.0)).astype(np.float32)
    assert np.array_equal(ieee.view(np.uint32), product.view(np.uint32))


def test_mean_as_reciprocal_product() -> None:
    rng = np.random.default_rng(5)
    widths = np.arange(1, 32769, dtype=np.int64)
    for chunk in np.array_split(widths, 16):
        # sums of squares span fp16's range: exact multiples of h, tiny and huge sums
        t = np.concatenate([
            (rng.integers(1, 1 << 20, size=(chunk.size, 8)) * chunk[:, None]).astype(np.float32),
            np.ldexp(rng.random((chunk.size, 24)), rng.integers(-48, 47, size=(chunk.size, 24))).astype(np.float32),
        ], axis=1)
        h = chunk[:, None].astype(np.float32)
        ieee = t / h
        product = (t.astype(np.float64) * (1.0 / chunk[:, None].astype(np.float64))).astype(np.float32)
        assert np.array_equal(ieee.view(np.uint32), product.view(np.uint32))
