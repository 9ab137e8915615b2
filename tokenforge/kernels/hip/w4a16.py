"""W4A16 linear and full-weight dequantization on gfx950 (counterpart of triton/w4a16.py).

``w4a16_gemm`` keeps the reference's signature, checks and messages (w4a16.py:149-232); the
config selects one of the compiled HIP kernels (``config.GemmConfig``). Split-K partials are
reduced on chip (gemv kernels) or by a fixed-order reduction kernel (LDS GEMM), so eager and
HIP-graph results are bit-identical.
"""

from __future__ import annotations

import ctypes

import torch

from tokenforge.kernels import _lib
from tokenforge.kernels.config import GemmConfig
from tokenforge.kernels.hip._common import on_device, ptr, require_gpu, stream_of


def _check_inputs(
    x: torch.Tensor,
    qweight_t: torch.Tensor,
    scales: torch.Tensor,
    qzeros: torch.Tensor,
    group_size: int,
) -> tuple[int, int, int]:
    """Shape, dtype and layout checks of w4a16.py:149-175 (same types and messages)."""
    if x.dim() != 2:
        raise ValueError(f"x must be 2-D [M, K], got shape {tuple(x.shape)}")
    if x.dtype != torch.float16:
        raise TypeError(f"x must be fp16, got {x.dtype}")
    m, k = x.shape
    n = qweight_t.shape[0]
    if qweight_t.shape[1] * 8 != k:
        raise ValueError(f"x has K={k} but qweight_t encodes K={qweight_t.shape[1] * 8}")
    if k % group_size != 0:
        raise ValueError(f"K={k} is not a multiple of group_size={group_size}")
    if tuple(scales.shape) != (k // group_size, n):
        raise ValueError(f"scales shape {tuple(scales.shape)} != {(k // group_size, n)}")
    if tuple(qzeros.shape) != (k // group_size, n // 8):
        raise ValueError(f"qzeros shape {tuple(qzeros.shape)} != {(k // group_size, n // 8)}")
    if qweight_t.dtype != torch.int32 or qzeros.dtype != torch.int32:
        raise TypeError("qweight_t and qzeros must be int32")
    if scales.dtype != torch.float16:
        raise TypeError(f"scales must be fp16, got {scales.dtype}")
    for name, t in (("qweight_t", qweight_t), ("scales", scales), ("qzeros", qzeros)):
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if x.stride(1) != 1:
        raise ValueError("x must be contiguous along K (stride(1) == 1)")
    return m, n, k


def to_c_config(cfg: GemmConfig) -> _lib.TfGemmConfig:
    return _lib.TfGemmConfig(
        _lib.KERNEL_IDS[cfg.kernel],
        cfg.block_m,
        cfg.block_n,
        cfg.block_k,
        cfg.split_k,
        cfg.num_warps,
        cfg.num_stages,
    )


def _aligned_rows(x: torch.Tensor) -> torch.Tensor:
    """x with 16-byte aligned rows (the kernels use 128-bit loads); copies only if needed."""
    if x.data_ptr() % 16 == 0 and (x.stride(0) % 8 == 0 or x.shape[0] <= 1):
        return x
    return x.clone(memory_format=torch.contiguous_format)


def workspace_bytes(m: int, n: int, k: int, group_size: int, cfg: GemmConfig) -> int:
    c = to_c_config(cfg)
    return int(_lib.lib().tf_w4a16_workspace_bytes(m, n, k, group_size, ctypes.byref(c)))


EPILOGUES = {"none": _lib.EPILOGUE_NONE, "residual": _lib.EPILOGUE_RESIDUAL, "silu_mul": _lib.EPILOGUE_SILU_MUL}


def w4a16_gemm(
    x: torch.Tensor,
    qweight_t: torch.Tensor,
    scales: torch.Tensor,
    qzeros: torch.Tensor,
    group_size: int,
    config: GemmConfig,
    bias: torch.Tensor | None = None,
) -> torch.Tensor:
    """``x [M, K] fp16`` @ dequant(W)^T (+ bias) -> ``[M, N] fp16`` (w4a16.py:178-232)."""
    return w4a16_gemm_ex(x, qweight_t, scales, qzeros, group_size, config, bias)


def _check_epilogue(m: int, n: int, epilogue: str,
                    residual: torch.Tensor | None) -> torch.Tensor | None:
    if epilogue not in EPILOGUES:
        raise ValueError(f"epilogue must be one of {sorted(EPILOGUES)}, got {epilogue!r}")
    if epilogue == "residual":
        if residual is None or tuple(residual.shape) != (m, n) or residual.dtype != torch.float16:
            raise ValueError(f"the residual epilogue needs an fp16 residual of shape {(m, n)}")
        if residual.stride(-1) != 1:
            residual = residual.contiguous()
    elif residual is not None:
        raise ValueError("residual is only used by the residual epilogue")
    if epilogue == "silu_mul" and n % 16:
        raise ValueError(f"the silu_mul epilogue needs N to be a multiple of 16, got {n}")
    return residual


def check_linear_args(
    x: torch.Tensor,
    qweight_t: torch.Tensor,
    scales: torch.Tensor,
    qzeros: torch.Tensor,
    group_size: int,
    bias: torch.Tensor | None,
    epilogue: str,
    residual: torch.Tensor | None,
) -> tuple[int, int, int, torch.Tensor | None, torch.Tensor | None]:
    """Every check of the W4A16 linear with an epilogue, on any device; returns ``(M, N, K)``
    and the bias and residual as the kernel reads them (contiguous along N)."""
    m, n, k = _check_inputs(x, qweight_t, scales, qzeros, group_size)
    if bias is not None:
        if tuple(bias.shape) != (n,):
            raise ValueError(f"bias shape {tuple(bias.shape)} != {(n,)}")
        if bias.dtype != torch.float16:
            raise TypeError(f"bias must be fp16, got {bias.dtype}")
        bias = bias.contiguous()
    return m, n, k, bias, _check_epilogue(m, n, epilogue, residual)


def check_w4a8_args(
    x8: torch.Tensor,
    x_scale: torch.Tensor,
    qweight_t: torch.Tensor,
    scales: torch.Tensor,
    qzeros: torch.Tensor,
    group_size: int,
    bias: torch.Tensor | None,
    epilogue: str,
    residual: torch.Tensor | None,
) -> tuple[int, int, int, torch.Tensor | None, torch.Tensor | None]:
    """Every check of the W4A8 linear, on any device; returns as :func:`check_linear_args`."""
    if x8.dim() != 2:
        raise ValueError(f"x8 must be 2-D [M, K], got shape {tuple(x8.shape)}")
    if x8.dtype != torch.float8_e4m3fn:
        raise TypeError(f"x8 must be float8_e4m3fn, got {x8.dtype}")
    m, k = x8.shape
    n = qweight_t.shape[0]
    # Shape checks of the fp16 path on a stand-in of x's shape.
    _check_inputs(torch.empty((m, k), dtype=torch.float16, device="meta"), qweight_t, scales, qzeros, group_size)
    if bias is not None:
        if tuple(bias.shape) != (n,) or bias.dtype != torch.float16:
            raise ValueError(f"bias must be fp16 of shape {(n,)}")
        bias = bias.contiguous()
    residual = _check_epilogue(m, n, epilogue, residual)
    _row_scales(x_scale, m)
    return m, n, k, bias, residual


def w4a16_gemm_ex(
    x: torch.Tensor,
    qweight_t: torch.Tensor,
    scales: torch.Tensor,
    qzeros: torch.Tensor,
    group_size: int,
    config: GemmConfig,
    bias: torch.Tensor | None = None,
    epilogue: str = "none",
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    """:func:`w4a16_gemm` with a fused epilogue (``tf_w4a16_linear_ex``):

    * ``"none"``: ``y``;
    * ``"residual"``: ``residual + y`` for an fp16 ``residual [M, N]`` (one fp16 add after the
      fp16 ``y``, as the unfused torch expression rounds);
    * ``"silu_mul"``: ``silu(y[:, :N/2]) * y[:, N/2:]`` -> ``[M, N/2]`` (torch's fp16 silu and
      multiply on the fp16 ``y``); N a multiple of 16.
    """
    m, n, k, bias, residual = check_linear_args(x, qweight_t, scales, qzeros, group_size, bias, epilogue, residual)
    config.validate(group_size)
    tensors = (x, qweight_t, scales, qzeros) + tuple(t for t in (bias, residual) if t is not None)
    dev = require_gpu("w4a16_gemm", *tensors)
    n_out = n // 2 if epilogue == "silu_mul" else n
    out = torch.empty((m, n_out), dtype=torch.float16, device=dev)
    if m == 0 or n == 0:
        return out
    x = _aligned_rows(x)
    ldx = x.stride(0) if m > 1 else k
    ldr = (residual.stride(0) if m > 1 else n) if residual is not None else 0
    code = EPILOGUES[epilogue]
    c = to_c_config(config)
    h = _lib.lib()
    need = int(h.tf_w4a16_workspace_bytes_ex(m, n, k, group_size, ctypes.byref(c), code))
    ws = torch.empty((max(need, 4) + 3) // 4, dtype=torch.float32, device=dev) if need else None
    with on_device(dev):
        rc = h.tf_w4a16_linear_ex(
            x.data_ptr(), ldx, qweight_t.data_ptr(), scales.data_ptr(), qzeros.data_ptr(),
            ptr(bias), out.data_ptr(), n_out, m, n, k, group_size, ctypes.byref(c), code,
            ptr(residual), ldr, ptr(ws), need, stream_of(dev),
        )
    _lib.check(rc, "tf_w4a16_linear_ex")
    return out


def check_dequant_inputs(qweight_t: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor,
                         group_size: int) -> tuple[int, int]:
    """The dequant kernel's dtype and shape checks; returns ``(N, K)``."""
    n = qweight_t.shape[0]
    k = qweight_t.shape[1] * 8
    if qweight_t.dtype != torch.int32 or qzeros.dtype != torch.int32:
        raise TypeError("qweight_t and qzeros must be int32")
    if scales.dtype != torch.float16:
        raise TypeError(f"scales must be fp16, got {scales.dtype}")
    if k % group_size != 0:
        raise ValueError(f"K={k} is not a multiple of group_size={group_size}")
    if tuple(scales.shape) != (k // group_size, n):
        raise ValueError(f"scales shape {tuple(scales.shape)} != {(k // group_size, n)}")
    if tuple(qzeros.shape) != (k // group_size, n // 8):
        raise ValueError(f"qzeros shape {tuple(qzeros.shape)} != {(k // group_size, n // 8)}")
    return n, k


def w4a16_dequant(
    qweight_t: torch.Tensor,
    scales: torch.Tensor,
    qzeros: torch.Tensor,
    group_size: int,
) -> torch.Tensor:
    """Tile-layout weights -> fp16 ``[N, K]`` (w4a16.py:235-264), bit-exact with dequantize_tf."""
    n, k = check_dequant_inputs(qweight_t, scales, qzeros, group_size)
    dev = require_gpu("w4a16_dequant", qweight_t, scales, qzeros)
    qweight_t, scales, qzeros = (t.contiguous() for t in (qweight_t, scales, qzeros))
    out = torch.empty((n, k), dtype=torch.float16, device=dev)
    if out.numel() == 0:
        return out
    with on_device(dev):
        rc = _lib.lib().tf_w4a16_dequant(
            qweight_t.data_ptr(), scales.data_ptr(), qzeros.data_ptr(), out.data_ptr(), n, k,
            group_size, stream_of(dev),
        )
    _lib.check(rc, "tf_w4a16_dequant")
    return out


def _row_scales(x_scale: torch.Tensor, m: int) -> tuple[torch.Tensor, int]:
    """``x_scale`` as the vector the kernel reads and its element stride (0: one scale for every
    row). The vector is contiguous, so its data pointer and stride describe the same memory."""
    if x_scale.dtype != torch.float32:
        raise TypeError(f"x_scale must be fp32, got {x_scale.dtype}")
    if x_scale.numel() == 1:
        return x_scale.reshape(1).contiguous(), 0
    if x_scale.numel() != m:
        raise ValueError(f"x_scale must hold one scale or one per row ({m}), got shape {tuple(x_scale.shape)}")
    return x_scale.reshape(m).contiguous(), 1


def w4a8_gemm_ex(
    x8: torch.Tensor,
    x_scale: torch.Tensor,
    qweight_t: torch.Tensor,
    scales: torch.Tensor,
    qzeros: torch.Tensor,
    group_size: int,
    config: GemmConfig,
    bias: torch.Tensor | None = None,
    epilogue: str = "none",
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    """W4A8: ``x_scale[m] * (e4m3(x8) @ dequant(W)^T) (+ bias)`` -> fp16, with the epilogues of
    :func:`w4a16_gemm_ex` (``tf_w4a8_linear_ex``). ``x8`` float8_e4m3fn ``[M, K]`` (as
    ``rmsnorm_fp8_quant`` returns it), ``x_scale`` fp32 with one value or one per row."""
    m, n, k, bias, residual = check_w4a8_args(x8, x_scale, qweight_t, scales, qzeros, group_size, bias, epilogue,
                                              residual)
    config.validate(group_size)
    x_scale, xs_stride = _row_scales(x_scale, m)
    tensors = (x8, x_scale, qweight_t, scales, qzeros) + tuple(t for t in (bias, residual) if t is not None)
    dev = require_gpu("w4a8_gemm", *tensors)
    n_out = n // 2 if epilogue == "silu_mul" else n
    out = torch.empty((m, n_out), dtype=torch.float16, device=dev)
    if m == 0 or n == 0:
        return out
    ldx8 = x8.stride(0) if m > 1 else k
    if x8.stride(-1) != 1 or ldx8 % 8 or x8.data_ptr() % 16:
        x8 = x8.clone(memory_format=torch.contiguous_format)  # a fresh, aligned allocation
        ldx8 = k
    ldr = (residual.stride(0) if m > 1 else n) if residual is not None else 0
    code = EPILOGUES[epilogue]
    c = to_c_config(config)
    h = _lib.lib()
    need = int(h.tf_w4a8_workspace_bytes_ex(m, n, k, group_size, ctypes.byref(c), code))
    ws = torch.empty((max(need, 4) + 3) // 4, dtype=torch.float32, device=dev) if need else None
    with on_device(dev):
        rc = h.tf_w4a8_linear_ex(
            x8.data_ptr(), ldx8, x_scale.data_ptr(), xs_stride, qweight_t.data_ptr(), scales.data_ptr(),
            qzeros.data_ptr(), ptr(bias), out.data_ptr(), n_out, m, n, k, group_size, ctypes.byref(c), code,
            ptr(residual), ldr, ptr(ws), need, stream_of(dev),
        )
    _lib.check(rc, "tf_w4a8_linear_ex")
    return out


def rmsnorm_fp8_w4a16_gemm_ex(
    x: torch.Tensor,
    norm_weight: torch.Tensor,
    eps: float,
    qweight_t: torch.Tensor,
    scales: torch.Tensor,
    qzeros: torch.Tensor,
    group_size: int,
    config: GemmConfig,
    bias: torch.Tensor | None = None,
    epilogue: str = "none",
) -> torch.Tensor:
    """``w4a16_gemm_ex(a, ...)`` with ``a`` the fp16 activation of ``rmsnorm_fp8_quant_dequant(x,
    norm_weight, eps)`` (dynamic scale), in one decode launch (``tf_rmsnorm_fp8_w4a16_linear``;
    no counterpart in the reference, which runs the norm and the linear as separate kernels).
    Same bits as the two calls. ``config`` must be the gemv stream form (``config.stream``, M
    <= 4); epilogue ``"none"`` or ``"silu_mul"``."""
    m, n, k = _check_inputs(x, qweight_t, scales, qzeros, group_size)
    config.validate(group_size)
    if not config.stream or config.split_k != 1:
        raise ValueError(f"the RMSNorm prologue runs in the gemv stream form (M <= 4, split_k 1), got config {config}")
    if epilogue not in ("none", "silu_mul"):
        raise ValueError(f"epilogue must be 'none' or 'silu_mul', got {epilogue!r}")
    if tuple(norm_weight.shape) != (k,):
        raise ValueError(f"norm weight shape {tuple(norm_weight.shape)} != {(k,)}")
    if norm_weight.dtype != torch.float16:
        raise TypeError(f"norm weight must be fp16, got {norm_weight.dtype}")
    if bias is not None:
        if tuple(bias.shape) != (n,):
            raise ValueError(f"bias shape {tuple(bias.shape)} != {(n,)}")
        if bias.dtype != torch.float16:
            raise TypeError(f"bias must be fp16, got {bias.dtype}")
        bias = bias.contiguous()
    if epilogue == "silu_mul" and n % 16:
        raise ValueError(f"the silu_mul epilogue needs N to be a multiple of 16, got {n}")
    tensors = (x, norm_weight, qweight_t, scales, qzeros) + (() if bias is None else (bias,))
    dev = require_gpu("rmsnorm_fp8_w4a16_gemm", *tensors)
    n_out = n // 2 if epilogue == "silu_mul" else n
    out = torch.empty((m, n_out), dtype=torch.float16, device=dev)
    if m == 0 or n == 0:
        return out
    x = _aligned_rows(x)
    if norm_weight.stride(0) != 1 or norm_weight.data_ptr() % 16:
        norm_weight = norm_weight.clone(memory_format=torch.contiguous_format)
    ldx = x.stride(0) if m > 1 else k
    c = to_c_config(config)
    with on_device(dev):
        rc = _lib.lib().tf_rmsnorm_fp8_w4a16_linear(
            x.data_ptr(), ldx, norm_weight.data_ptr(), float(eps), qweight_t.data_ptr(), scales.data_ptr(),
            qzeros.data_ptr(), ptr(bias), out.data_ptr(), n_out, m, n, k, group_size, ctypes.byref(c),
            EPILOGUES[epilogue], stream_of(dev),
        )
    _lib.check(rc, "tf_rmsnorm_fp8_w4a16_linear")
    return out
