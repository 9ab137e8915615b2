"""Deterministic test cases shared by the numerics tests and the tolerance calibration.

Same generators and seeds as the reference's tests/numerics/cases.py:16-37: seeds are
``zlib.crc32(repr(parts))`` into ``torch.Generator``; weights are ``awq_quantize(randn * 0.02)``
(here the oracle's restatement), so the inputs are the reference's own test inputs.
"""

from __future__ import annotations

import functools
import zlib

import numpy as np
import torch

from oracle import pack as opack
from tokenforge.kernels.pack import W4A16Weights

GROUP_SIZE = 128
TEST_SEEDS = (0,)
CALIBRATION_SEEDS = (0, 1, 2, 3, 4)


def _seed(*parts: object) -> int:
    return zlib.crc32(repr(parts).encode())


@functools.lru_cache(maxsize=16)
def layer_weights(n: int, k: int, seed: int, group_size: int = GROUP_SIZE) -> opack.W4A16Weights:
    """Oracle-layout (numpy) weights of one seeded layer."""
    gen = torch.Generator().manual_seed(_seed("w", n, k, seed, group_size))
    weight = (torch.randn((n, k), generator=gen) * 0.02).numpy()
    return opack.pack_awq(*opack.awq_quantize(weight, group_size), group_size)


def activations(m: int, k: int, seed: int) -> torch.Tensor:
    gen = torch.Generator().manual_seed(_seed("x", m, k, seed))
    return torch.randn((m, k), generator=gen).to(torch.float16)


def bias(n: int, seed: int) -> torch.Tensor:
    gen = torch.Generator().manual_seed(_seed("b", n, seed))
    return (torch.randn((n,), generator=gen) * 0.1).to(torch.float16)


def on_device(w: opack.W4A16Weights, device: torch.device) -> W4A16Weights:
    """Oracle numpy weights (TokenForge layout) -> product weights on ``device``, in the tile
    layout the kernels read (laid out by the oracle's restatement of it)."""
    qw, sc, qz = opack.tile_pack(w.qweight_t, w.scales, w.qzeros, w.group_size)
    return W4A16Weights(
        torch.from_numpy(np.ascontiguousarray(qw)).to(device),
        torch.from_numpy(np.ascontiguousarray(sc)).to(device),
        torch.from_numpy(np.ascontiguousarray(qz)).to(device),
        w.group_size,
    )


def baseline_layer(n: int, k: int, seed: int, group_size: int = GROUP_SIZE):
    """BASELINE configs 1/3/4 weights: nibbles and zero-points uniform in [0, 15], fp16 scales
    uniform in [1e-3, 1e-2]; AWQ ``(qweight, qzeros, scales)`` as numpy arrays."""
    gen = torch.Generator().manual_seed(_seed("baseline", n, k, seed, group_size))
    intweight = torch.randint(0, 16, (k, n), generator=gen, dtype=torch.int32).numpy()
    zeros = torch.randint(0, 16, (k // group_size, n), generator=gen, dtype=torch.int32).numpy()
    scales = (torch.rand((k // group_size, n), generator=gen) * 9e-3 + 1e-3).to(torch.float16).numpy()
    qweight, qzeros = opack.awq_pack(intweight, zeros)
    return qweight, qzeros, scales
