"""The native seam the reference planned as ``tokenforge.kernels._C`` (ops.py:34-40, :86-88).

The reference's op would call ``_C.w4a16_gemv(x2, qweight_t, scales, qzeros, bias,
group_size)`` for decode-sized M; here that call runs the gfx950 decode kernel with the
bucket's tuned (or default) configuration.
"""

from __future__ import annotations

import torch

from tokenforge.kernels import autotune
from tokenforge.kernels.config import GEMV_MAX_M, m_bucket
from tokenforge.kernels.device import gpu_identity
from tokenforge.kernels.hip.w4a16 import w4a16_gemm


def w4a16_gemv(
    x2: torch.Tensor,
    qweight_t: torch.Tensor,
    scales: torch.Tensor,
    qzeros: torch.Tensor,
    bias: torch.Tensor | None,
    group_size: int,
) -> torch.Tensor:
    """``x2 [M, K]`` fp16, M <= 32 -> ``[M, N]`` fp16 through the streaming decode kernel."""
    m, k = x2.shape
    if not 1 <= m <= GEMV_MAX_M:
        raise ValueError(f"w4a16_gemv serves 1 <= M <= {GEMV_MAX_M}, got M={m}")
    n = qweight_t.shape[0]
    cfg = autotune.lookup(gpu_identity(x2.device), m_bucket(m), n, k, group_size)
    return w4a16_gemm(x2, qweight_t, scales, qzeros, group_size, cfg, bias)
