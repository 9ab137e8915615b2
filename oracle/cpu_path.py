"""Torch-CPU restatement of the reference's CPU execution path, for the timed CPU baseline.

Test infrastructure only (see ``oracle/__init__.py``). ``w4a16_torch_cpu`` follows
reference.py:24-32 as ops.py:79-81 runs it when no kernel can run: dequantize the whole
weight on every call (pack.py:189-194), fp32 matmul, add bias in fp32, cast to fp16. It uses
torch's intra-op thread pool, so its thread count is ``torch.get_num_threads()``.
"""

from __future__ import annotations

import torch

_SHIFTS = torch.tensor([4 * j for j in (0, 4, 1, 5, 2, 6, 3, 7)], dtype=torch.int32)  # 4*AWQ_REVERSE_ORDER


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    """pack.py:57-67."""
    values = (packed.unsqueeze(-1) >> _SHIFTS) & 0xF
    return values.reshape(*packed.shape[:-1], packed.shape[-1] * 8)


def dequantize_tf(qweight_t: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor, group_size: int) -> torch.Tensor:
    """pack.py:189-194: TokenForge layout -> fp16 [N, K]."""
    q = unpack_int4(qweight_t)
    z = unpack_int4(qzeros).repeat_interleave(group_size, dim=0).t()
    s = scales.repeat_interleave(group_size, dim=0).t()
    return (q - z).to(torch.float16) * s


def w4a16_torch_cpu(
    x: torch.Tensor,
    qweight_t: torch.Tensor,
    scales: torch.Tensor,
    qzeros: torch.Tensor,
    group_size: int,
    bias: torch.Tensor | None = None,
) -> torch.Tensor:
    """reference.py:24-32 on CPU tensors."""
    w = dequantize_tf(qweight_t, scales, qzeros, group_size)
    y = x.to(torch.float32) @ w.to(torch.float32).t()
    if bias is not None:
        y = y + bias.to(torch.float32)
    return y.to(x.dtype)


_AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


def pack_int4(values: torch.Tensor) -> torch.Tensor:
    """pack.py:42-54 (without the range check): word = sum_i v[..., AWQ_ORDER[i]] << 4i in
    int64, wrapped to the int32 bit pattern."""
    *lead, n = values.shape
    v = values.to(torch.int64).reshape(*lead, n // 8, 8)
    word = torch.zeros(v.shape[:-1], dtype=torch.int64)
    for nibble, offset in enumerate(_AWQ_ORDER):
        word |= v[..., offset] << (4 * nibble)
    return word.to(torch.int32)


def repack_awq_to_tf_cpu(qweight: torch.Tensor) -> torch.Tensor:
    """pack.py:141-143 on CPU tensors: pack_int4(awq_unpack(qweight).t())."""
    return pack_int4(unpack_int4(qweight).t().contiguous())


def rmsnorm_fp8_torch_cpu(x: torch.Tensor, weight: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """reference.py:35-56 on CPU tensors (dynamic per-token scale): HF RMSNorm in fp32 rounded
    to fp16, times the fp16 weight, then per-row scale = max(amax / 448, 1 / (448 * 512)) and
    the e4m3fn cast of y / scale."""
    xf = x.to(torch.float32)
    var = xf.pow(2).mean(-1, keepdim=True)
    y = (xf * torch.rsqrt(var + eps)).to(torch.float16) * weight
    amax = y.abs().amax(-1, keepdim=True).to(torch.float32)
    scale = torch.clamp(amax / 448.0, min=1.0 / (448.0 * 512.0))
    q = (y.to(torch.float32) / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q, scale
