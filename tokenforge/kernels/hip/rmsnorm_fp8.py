"""Fused RMSNorm + FP8 (e4m3fn) quantization on gfx950 (counterpart of triton/rmsnorm_fp8.py).

Each row is read from HBM once, by one workgroup ("row_per_block", the default) or by one wave
("row_per_wave"); ``form`` picks the kernel form explicitly (same bits either way). Semantics follow
reference.py:35-56 (HF Qwen2 RMSNorm, then per-token dynamic or static per-tensor e4m3
quantization with an IEEE division and round-to-nearest-even onto the e4m3 grid).
"""

from __future__ import annotations

import torch

from tokenforge.kernels import _lib
from tokenforge.kernels.hip._common import on_device, require_gpu, stream_of

FP8_E4M3_MAX = 448.0
MIN_SCALE = 1.0 / (FP8_E4M3_MAX * 512.0)
FORMS = {"auto": 0, "row_per_block": 1, "row_per_wave": 2}  # TF_NORM_* of the C header


def rmsnorm_fp8_quant(
    x: torch.Tensor,
    weight: torch.Tensor,
    eps: float,
    scale: torch.Tensor | None = None,
    *,
    form: str = "auto",
) -> tuple[torch.Tensor, torch.Tensor]:
    """``x [T, H]`` -> ``(q [T, H] float8_e4m3fn, scale)`` (rmsnorm_fp8.py:76-117).

    ``scale`` is ``[T, 1]`` fp32 for dynamic per-token quantization, or the given ``[1]``
    fp32 tensor for static per-tensor quantization (read, not written).
    """
    q, s, _ = _launch(x, weight, eps, scale, dequant=False, form=form)
    return q, s


def rmsnorm_fp8_quant_dequant(
    x: torch.Tensor,
    weight: torch.Tensor,
    eps: float,
    scale: torch.Tensor | None = None,
    *,
    form: str = "auto",
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """:func:`rmsnorm_fp8_quant` plus ``a [T, H]`` fp16 = ``(q.to(float32) * scale).to(float16)``,
    the fp16 activation a W4A16 linear reads when it is fed from the codes, in the same launch
    (no counterpart in the reference, which would run that expression as separate torch ops)."""
    q, s, a = _launch(x, weight, eps, scale, dequant=True, form=form)
    assert a is not None
    return q, s, a


def check_inputs(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor | None) -> tuple[int, int]:
    """Shape, layout and dtype checks of the norm; returns ``(T, H)``."""
    if x.dim() != 2:
        raise ValueError(f"x must be 2-D [T, H], got {tuple(x.shape)}")
    t, h = x.shape
    if tuple(weight.shape) != (h,):
        raise ValueError(f"weight shape {tuple(weight.shape)} != {(h,)}")
    if x.stride(1) != 1:
        raise ValueError("x must be contiguous along H")
    if x.dtype != torch.float16 or weight.dtype != torch.float16:
        raise TypeError(f"x and weight must be fp16, got {x.dtype} and {weight.dtype}")
    if scale is not None and (scale.numel() != 1 or scale.dtype != torch.float32):
        raise ValueError("static scale must be a single fp32 element")
    return t, h


def _launch(
    x: torch.Tensor, weight: torch.Tensor, eps: float, scale: torch.Tensor | None, dequant: bool,
    form: str = "auto",
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    if form not in FORMS:
        raise ValueError(f"form must be one of {sorted(FORMS)}, got {form!r}")
    t, h = check_inputs(x, weight, scale)
    dev = require_gpu("rmsnorm_fp8_quant", x, weight, *(() if scale is None else (scale,)))
    weight = weight.contiguous()
    out = torch.empty((t, h), dtype=torch.float8_e4m3fn, device=dev)
    static = scale is not None
    scale_out = scale if static else torch.empty((t, 1), dtype=torch.float32, device=dev)
    a = torch.empty((t, h), dtype=torch.float16, device=dev) if dequant else None
    if t == 0 or h == 0:
        return out, scale_out, a
    ldx = x.stride(0) if t > 1 else h
    with on_device(dev):
        rc = _lib.lib().tf_rmsnorm_fp8_quant_ex(
            x.data_ptr(), ldx, weight.data_ptr(), out.data_ptr(), h, scale_out.data_ptr(),
            1 if static else 0, 0 if a is None else a.data_ptr(), h, t, h, float(eps), FORMS[form],
            stream_of(dev),
        )
    _lib.check(rc, "tf_rmsnorm_fp8_quant_ex")
    return out, scale_out, a


def e4m3_encode(values: torch.Tensor) -> torch.Tensor:
    """The kernel's e4m3fn encoder on an fp32 tensor with |v| <= 448 (test hook)."""
    if values.dtype != torch.float32:
        raise TypeError(f"values must be fp32, got {values.dtype}")
    dev = require_gpu("e4m3_encode", values)
    v = values.contiguous()
    out = torch.empty(v.shape, dtype=torch.float8_e4m3fn, device=dev)
    if v.numel() == 0:
        return out
    with on_device(dev):
        rc = _lib.lib().tf_e4m3_encode(v.data_ptr(), out.data_ptr(), v.numel(), stream_of(dev))
    _lib.check(rc, "tf_e4m3_encode")
    return out
