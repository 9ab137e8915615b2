"""AWQ checkpoint format, the TokenForge layout and the gfx950 tile layout (pack.py:1-194).

Three layouts of one W4A16 layer (K input features, N output features, group size G):

* **AWQ GEMM format** (AutoAWQ ``WQLinear_GEMM``, what checkpoints hold): ``qweight`` int32
  ``[K, N/8]`` packed along N, ``qzeros`` int32 ``[K/G, N/8]``, ``scales`` fp16 ``[K/G, N]``.
  A word holds eight 4-bit values in the nibble order ``AWQ_ORDER`` (offsets ``2j, 2j+1`` in
  nibbles ``j, j+4``), so masking a word with ``0x000F000F`` and OR-ing the fp16 exponent
  ``0x6400`` gives the fp16 pair ``(1024 + q[2j], 1024 + q[2j+1])``.
* **TokenForge layout** (the reference's, bit-identical here): ``qweight_t`` int32 ``[N, K/8]``
  packed along K (:func:`repack_awq_to_tf`), scales and zero points as in AWQ.
* **gfx950 tile layout** (what :func:`pack_awq` returns and every kernel reads): the same three
  shapes and dtypes, with rows grouped in tiles of 16. Each 16-row x 128-K step of
  ``qweight_t`` is one contiguous 1 KB block of 16-byte chunks (32 K values of one row), in
  which lane ``16 g + c`` of a wave finds the MFMA B operand of column ``c``, K block ``g``;
  a tile's scales and zero points are contiguous, group after group. The exact index maps are
  in ``tokenforge_amd/csrc/tile_layout.h``.

Dequantization is ``w[k, n] = fp16(q[k, n] - z[k // G, n]) * s[k // G, n]`` (one rounding).

Every tensor-producing function runs a HIP kernel on a gfx950 GPU. These are load-time
functions, so they also accept host tensors (as the reference's callers pass them): the
inputs are copied to the current GPU, the kernel runs there, and the results come back on
the inputs' device. Without a visible GPU, host tensors take the torch route
(``tokenforge.kernels.host``), which gives the same bits.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from tokenforge.kernels.hip import layout as _layout

AWQ_ORDER: tuple[int, ...] = (0, 2, 4, 6, 1, 3, 5, 7)
"""``AWQ_ORDER[i]`` is the column offset (0..7) stored in bits ``4i..4i+3`` of an AWQ word."""

AWQ_REVERSE_ORDER: tuple[int, ...] = (0, 4, 1, 5, 2, 6, 3, 7)
"""The nibble that stores column offset ``j``: the inverse permutation, ``(j % 2) * 4 + j // 2``."""

PACK_FACTOR = 8
SUPPORTED_GROUP_SIZES: tuple[int, ...] = (32, 64, 128)


def pack_int4(values: torch.Tensor) -> torch.Tensor:
    """Eight 4-bit values of the last dimension per int32 word, placed in the AWQ nibble order."""
    return _layout.pack_int4(values)


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    """Every nibble of every word back in column order, as int32 in [0, 15] (undoes :func:`pack_int4`)."""
    return _layout.unpack_int4(packed)


def awq_pack(intweight: torch.Tensor, zeros: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """AWQ ``(qweight, qzeros)`` from 4-bit ``intweight [K, N]`` and ``zeros [K // G, N]``."""
    return pack_int4(intweight), pack_int4(zeros)


def awq_unpack(qweight: torch.Tensor) -> torch.Tensor:
    """The 4-bit values of an AWQ ``qweight [K, N // 8]`` (or ``qzeros``) as int32 ``[K, N]``."""
    return unpack_int4(qweight)


def awq_quantize(weight: torch.Tensor, group_size: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Min-max asymmetric int4 quantization of an ``nn.Linear`` weight ``[N, K]`` into AWQ format
    (AutoAWQ's rounding rules): ``(qweight [K, N/8], qzeros [K/G, N/8], scales [K/G, N] fp16)``.
    A fixture generator for tests and benchmarks; production loads real AWQ checkpoints."""
    return _layout.awq_quantize(weight, group_size)


@dataclass(frozen=True)
class W4A16Weights:
    """One linear layer's weights as the kernels read them (the gfx950 tile layout when built
    by :func:`pack_awq`); the shapes and dtypes are the reference's."""

    qweight_t: torch.Tensor  # int32 [N, K // 8]
    scales: torch.Tensor  # fp16 [K // G, N]
    qzeros: torch.Tensor  # int32 [K // G, N // 8]
    group_size: int

    @property
    def n(self) -> int:
        return int(self.qweight_t.shape[0])

    @property
    def k(self) -> int:
        return int(self.qweight_t.shape[1]) * PACK_FACTOR


def repack_awq_to_tf(qweight: torch.Tensor) -> torch.Tensor:
    """AWQ ``qweight [K, N // 8]`` -> TokenForge ``qweight_t [N, K // 8]`` (bit-exact)."""
    return _layout.awq_to_tf(qweight)


def repack_tf_to_awq(qweight_t: torch.Tensor) -> torch.Tensor:
    """TokenForge ``qweight_t [N, K // 8]`` back to AWQ ``qweight [K, N // 8]`` (bit-exact)."""
    return _layout.tf_to_awq(qweight_t)


def validate_awq(
    qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor, group_size: int
) -> None:
    """Check shapes, dtypes and group size of one AWQ layer; ``ValueError`` names the first violation."""
    if qweight.dtype != torch.int32 or qzeros.dtype != torch.int32:
        raise ValueError("qweight and qzeros must be int32")
    if scales.dtype != torch.float16:
        raise ValueError(f"scales must be fp16, got {scales.dtype}")
    if group_size not in SUPPORTED_GROUP_SIZES:
        raise ValueError(f"group_size {group_size} not in {SUPPORTED_GROUP_SIZES}")
    k, n8 = qweight.shape
    n = n8 * PACK_FACTOR
    if k % group_size != 0:
        raise ValueError(f"K={k} is not a multiple of group_size={group_size}")
    if tuple(qzeros.shape) != (k // group_size, n8):
        raise ValueError(f"qzeros shape {tuple(qzeros.shape)} != {(k // group_size, n8)}")
    if tuple(scales.shape) != (k // group_size, n):
        raise ValueError(f"scales shape {tuple(scales.shape)} != {(k // group_size, n)}")


def pack_awq(
    qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor, group_size: int
) -> W4A16Weights:
    """Load-time conversion of one AWQ layer into the gfx950 tile layout: the GPU repack to the
    TokenForge layout, then the tile permutation of the weights, scales and zero points."""
    validate_awq(qweight, qzeros, scales, group_size)
    qw, sc, qz = _layout.tile_pack(repack_awq_to_tf(qweight), scales, qzeros, group_size)
    return W4A16Weights(qweight_t=qw, scales=sc, qzeros=qz, group_size=group_size)


def unpack_to_awq(weights: W4A16Weights) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Inverse of :func:`pack_awq`: returns ``(qweight, qzeros, scales)`` in AWQ format."""
    qw, sc, qz = _layout.tile_unpack(weights.qweight_t, weights.scales, weights.qzeros, weights.group_size)
    return repack_tf_to_awq(qw), qz, sc


def dequantize_tf(weights: W4A16Weights) -> torch.Tensor:
    """Tile-layout weights -> fp16 ``[N, K]`` (the ``nn.Linear.weight`` layout)."""
    from tokenforge.kernels import host
    from tokenforge.kernels.hip._common import host_route, load_time_devices
    from tokenforge.kernels.hip.w4a16 import w4a16_dequant

    if host_route(weights.qweight_t, weights.scales, weights.qzeros):
        return host.dequantize(weights.qweight_t, weights.scales, weights.qzeros, weights.group_size)
    run, home = load_time_devices("dequantize_tf", weights.qweight_t, weights.scales, weights.qzeros)
    qw, sc, qz = (t.to(run) for t in (weights.qweight_t, weights.scales, weights.qzeros))
    return w4a16_dequant(qw, sc, qz, weights.group_size).to(home)


def awq_dequantize(
    qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor, group_size: int
) -> torch.Tensor:
    """fp16 ``[K, N]`` weights of an AWQ layer, each ``fp16(q - z) * s`` rounded once, as the kernels do."""
    w = pack_awq(qweight, qzeros, scales, group_size)
    return dequantize_tf(w).t().contiguous()
