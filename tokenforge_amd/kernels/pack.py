"""AWQ GEMM-format packing and the TokenForge kernel layout (pack.py:1-194 in the reference).

AWQ GEMM layout (AutoAWQ ``WQLinear_GEMM``), the on-disk format every engine reads:

* ``qweight``: int32 ``[K, N // 8]``. Eight 4-bit weights per word, packed along N.
* ``qzeros``:  int32 ``[K // G, N // 8]``. Zero-points, packed the same way.
* ``scales``:  fp16  ``[K // G, N]``.

Inside a word, nibble ``i`` holds offset ``AWQ_ORDER[i]``: offsets ``(2j, 2j+1)`` sit in
nibbles ``(j, j+4)``, so ``word & 0x000F000F`` OR-ed with the fp16 pattern ``0x6400`` is the
fp16x2 pair ``(1024 + q[2j], 1024 + q[2j+1])`` that gfx950's packed-fp16 VALU consumes.

TokenForge layout (what the kernels read), bit-identical to the reference's:

* ``qweight_t``: int32 ``[N, K // 8]``, packed along K with the same nibble interleave. A
  lane that owns output row ``n`` streams contiguous K with 128-bit loads.
* ``scales`` and ``qzeros`` stay in AWQ layout.

Dequantization is ``w[k, n] = fp16(q[k, n] - z[k // G, n]) * s[k // G, n]`` (one rounding).

Every tensor-producing function here runs a HIP kernel on a gfx950 GPU tensor; CPU tensors
raise (the CPU restatement used to check these kernels lives in the repository's ``oracle``
test package, not here).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from tokenforge_amd.kernels.hip import layout as _layout

AWQ_ORDER: tuple[int, ...] = (0, 2, 4, 6, 1, 3, 5, 7)
"""Nibble ``i`` of a packed word holds offset ``AWQ_ORDER[i]``."""

AWQ_REVERSE_ORDER: tuple[int, ...] = (0, 4, 1, 5, 2, 6, 3, 7)
"""Offset ``j`` lives in nibble ``AWQ_REVERSE_ORDER[j]``. Equals ``(j % 2) * 4 + j // 2``."""

PACK_FACTOR = 8
SUPPORTED_GROUP_SIZES: tuple[int, ...] = (32, 64, 128)


def pack_int4(values: torch.Tensor) -> torch.Tensor:
    """Pack unsigned 4-bit values along the last dim into int32 words, AWQ interleave."""
    return _layout.pack_int4(values)


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    """Inverse of :func:`pack_int4`. Returns int32 values in [0, 15]."""
    return _layout.unpack_int4(packed)


def awq_pack(intweight: torch.Tensor, zeros: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Pack ``intweight [K, N]`` and ``zeros [K // G, N]`` (both in [0, 15]) into AWQ format."""
    return pack_int4(intweight), pack_int4(zeros)


def awq_unpack(qweight: torch.Tensor) -> torch.Tensor:
    """AWQ ``qweight [K, N // 8]`` -> int32 ``[K, N]``. Also works for ``qzeros``."""
    return unpack_int4(qweight)


@dataclass(frozen=True)
class W4A16Weights:
    """One linear layer's weights in TokenForge layout."""

    qweight_t: torch.Tensor  # int32 [N, K // 8], packed along K
    scales: torch.Tensor  # fp16 [K // G, N]
    qzeros: torch.Tensor  # int32 [K // G, N // 8], AWQ layout
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
    """Inverse of :func:`repack_awq_to_tf`."""
    return _layout.tf_to_awq(qweight_t)


def validate_awq(
    qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor, group_size: int
) -> None:
    """Raise ``ValueError`` with a precise reason if tensors are not a valid AWQ layer."""
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
    """Load-time conversion of one AWQ layer into the TokenForge layout (GPU repack)."""
    validate_awq(qweight, qzeros, scales, group_size)
    return W4A16Weights(
        qweight_t=repack_awq_to_tf(qweight),
        scales=scales.contiguous(),
        qzeros=qzeros.contiguous(),
        group_size=group_size,
    )


def unpack_to_awq(weights: W4A16Weights) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Inverse of :func:`pack_awq`: returns ``(qweight, qzeros, scales)``."""
    return repack_tf_to_awq(weights.qweight_t), weights.qzeros, weights.scales


def dequantize_tf(weights: W4A16Weights) -> torch.Tensor:
    """TokenForge layout -> fp16 ``[N, K]`` (the ``nn.Linear.weight`` layout)."""
    from tokenforge_amd.kernels.hip.w4a16 import w4a16_dequant

    return w4a16_dequant(weights.qweight_t, weights.scales, weights.qzeros, weights.group_size)


def awq_dequantize(
    qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor, group_size: int
) -> torch.Tensor:
    """AWQ format -> fp16 ``[K, N]`` with the single-rounding rule shared by every kernel."""
    w = pack_awq(qweight, qzeros, scales, group_size)
    return dequantize_tf(w).t().contiguous()
