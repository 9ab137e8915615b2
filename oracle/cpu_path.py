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
