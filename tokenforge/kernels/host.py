"""The torch route for host (CPU) tensors.

The reference sends a tensor that is not on the GPU through device-agnostic torch code: its
dispatcher decides ``torch_reference`` (dispatch.py:90-91), the linear then multiplies by the
dequantized weights in fp32 (ops.py:79-81, reference.py:24-32), the norm runs the HF RMSNorm
and the e4m3 quantization in torch (ops.py:132-133, reference.py:35-56), and the layout
functions are torch expressions (pack.py:42-194).

This module is that route here. The ops send host tensors to it, and the load-time layout
functions do so when no GPU is visible (with a GPU they copy host tensors to it, run the
kernels and copy the results back: the integer layouts come back as the same bits). A GPU
tensor never comes here: a GPU call without the kernel library raises.

The weights are in the gfx950 tile layout that :func:`tokenforge.kernels.pack.pack_awq`
produces (the chunk, scale and zero-point maps of ``tokenforge_amd/csrc/tile_layout.h``, stated
again below as index arithmetic over whole tensors).
"""

from __future__ import annotations

import torch

PACK_FACTOR = 8
FP8_E4M3_MAX = 448.0
MIN_SCALE = 1.0 / (FP8_E4M3_MAX * 512.0)


def _offset_shifts(device: torch.device) -> torch.Tensor:
    """Bit position of column offset j (0..7) inside an AWQ word: column offset j is stored
    in nibble ``(j % 2) * 4 + j // 2`` (even offsets in the low half, odd in the high)."""
    return torch.tensor([4 * ((j % 2) * 4 + j // 2) for j in range(PACK_FACTOR)], dtype=torch.int64,
                        device=device)


# ----------------------------------------------------------------------------- int4 packing


def pack_int4(values: torch.Tensor) -> torch.Tensor:
    """Every eight values of the last dimension into one int32 word, AWQ nibble order."""
    if values.shape[-1] % PACK_FACTOR != 0:
        raise ValueError(f"last dim {values.shape[-1]} is not a multiple of {PACK_FACTOR}")
    v = values.to(torch.int64)
    if v.numel() and bool(((v < 0) | (v > 15)).any()):
        raise ValueError("int4 values must lie in [0, 15]")
    *lead, n = v.shape
    fields = v.reshape(*lead, n // PACK_FACTOR, PACK_FACTOR) << _offset_shifts(v.device)
    word = fields.sum(dim=-1)  # disjoint bit fields: the sum is their OR, below 2^32
    return torch.where(word >= 2**31, word - 2**32, word).to(torch.int32)


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    """The eight 4-bit values of every word, in column order, as int32 in [0, 15]."""
    if packed.dtype != torch.int32:
        raise TypeError(f"packed tensor must be int32, got {packed.dtype}")
    nibbles = (packed.to(torch.int64).unsqueeze(-1) >> _offset_shifts(packed.device)) & 0xF
    return nibbles.reshape(*packed.shape[:-1], packed.shape[-1] * PACK_FACTOR).to(torch.int32)


def transpose_packed(src: torch.Tensor) -> torch.Tensor:
    """AWQ ``qweight [K, N/8]`` <-> TokenForge ``qweight_t [N, K/8]``: unpack, transpose and
    pack again, which is the conversion in either direction."""
    if src.dtype != torch.int32:
        raise TypeError(f"packed tensor must be int32, got {src.dtype}")
    if src.dim() != 2:
        raise ValueError(f"packed weight must be 2-D, got shape {tuple(src.shape)}")
    if src.shape[0] % PACK_FACTOR != 0:
        raise ValueError(f"{src.shape[0]} rows is not a multiple of {PACK_FACTOR}")
    return pack_int4(unpack_int4(src).t())


# ----------------------------------------------------------------------------- tile layout


def _tile_rows(n_total: int, t: torch.Tensor) -> torch.Tensor:
    """Rows of tile t: 16, or fewer for the last tile of an N that is not a multiple of 16."""
    return (n_total - 16 * t).clamp(max=16)


def chunk_positions(n_total: int, q_total: int) -> torch.Tensor:
    """``[N, K/32]``: where 16-byte chunk q (K offsets 32q..32q+31) of row n goes. A tile of
    r rows owns 16·Q consecutive chunks; inside it, 128-wide K step j is the block of 4r chunks
    starting at 4rj, ordered chunk-in-step major, row minor."""
    n = torch.arange(n_total, dtype=torch.int64)[:, None]
    q = torch.arange(q_total, dtype=torch.int64)[None, :]
    t, c = n // 16, n % 16
    r = _tile_rows(n_total, t)
    return 16 * q_total * t + 4 * r * (q // 4) + r * (q % 4) + c


def scale_positions(n_total: int, p_total: int) -> torch.Tensor:
    """``[K/G, N]``: where the scale of group p, row n goes (a tile's groups one after another,
    each group's r scales contiguous)."""
    p = torch.arange(p_total, dtype=torch.int64)[:, None]
    n = torch.arange(n_total, dtype=torch.int64)[None, :]
    t = n // 16
    return 16 * p_total * t + p * _tile_rows(n_total, t) + n % 16


def zero_positions(n_total: int, p_total: int) -> torch.Tensor:
    """``[K/G, N/8]``: where zero-point word w (rows 8w..8w+7) of group p goes."""
    p = torch.arange(p_total, dtype=torch.int64)[:, None]
    w = torch.arange(n_total // PACK_FACTOR, dtype=torch.int64)[None, :]
    t = w // 2
    return 2 * p_total * t + p * (_tile_rows(n_total, t) // PACK_FACTOR) + (w - 2 * t)


def _tile_maps(qweight_t: torch.Tensor, group_size: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    n, words = qweight_t.shape
    k = words * PACK_FACTOR
    return chunk_positions(n, k // 32).reshape(-1), scale_positions(n, k // group_size).reshape(-1), \
        zero_positions(n, k // group_size).reshape(-1)


def tile_pack(qweight_t: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor,
              group_size: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """TokenForge layout -> gfx950 tile layout (same shapes and dtypes; positions permuted)."""
    cpos, spos, zpos = _tile_maps(qweight_t, group_size)
    qw = torch.empty_like(qweight_t)
    sc = torch.empty_like(scales)
    qz = torch.empty_like(qzeros)
    qw.view(-1, 4)[cpos] = qweight_t.contiguous().view(-1, 4)
    sc.view(-1)[spos] = scales.contiguous().view(-1)
    qz.view(-1)[zpos] = qzeros.contiguous().view(-1)
    return qw, sc, qz


def tile_unpack(qweight_t: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor,
                group_size: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """gfx950 tile layout -> TokenForge layout (the inverse permutation of :func:`tile_pack`)."""
    cpos, spos, zpos = _tile_maps(qweight_t, group_size)
    qw = qweight_t.contiguous().view(-1, 4)[cpos].reshape(qweight_t.shape)
    sc = scales.contiguous().view(-1)[spos].reshape(scales.shape)
    qz = qzeros.contiguous().view(-1)[zpos].reshape(qzeros.shape)
    return qw, sc, qz


# ----------------------------------------------------------------------------- quantize / dequantize


def awq_quantize(weight: torch.Tensor, group_size: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Min-max asymmetric int4 of ``weight [N, K]`` per group of K, AutoAWQ's rounding: the
    scale is ``fp16(max(max - min, 1e-5) / 15)``, the zero point ``clamp(-round(min / s), 0,
    15)`` and the code ``clamp(round(w / s) + z, 0, 15)`` (fp32, IEEE division, ties to even).
    Returns AWQ ``(qweight [K, N/8], qzeros [K/G, N/8], scales [K/G, N] fp16)``."""
    n, k = weight.shape
    groups = weight.to(torch.float32).reshape(n, k // group_size, group_size)
    hi = groups.amax(dim=-1, keepdim=True)
    lo = groups.amin(dim=-1, keepdim=True)
    step = ((hi - lo).clamp(min=1e-5) / 15).to(torch.float16).to(torch.float32)
    zero = (-torch.round(lo / step)).clamp(0, 15)
    codes = (torch.round(groups / step) + zero).clamp(0, 15).reshape(n, k)
    qweight = pack_int4(codes.t().to(torch.int32))
    qzeros = pack_int4(zero[..., 0].t().to(torch.int32))
    return qweight, qzeros, step[..., 0].t().to(torch.float16).contiguous()


def dequantize(qweight_t: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor,
               group_size: int) -> torch.Tensor:
    """Tile-layout weights -> fp16 ``[N, K]``, each element ``fp16(q - z) * s`` rounded once."""
    qw, sc, qz = tile_unpack(qweight_t, scales, qzeros, group_size)
    q = unpack_int4(qw)  # [N, K]
    z = unpack_int4(qz).repeat_interleave(group_size, dim=0).t()  # [N, K]
    s = sc.repeat_interleave(group_size, dim=0).t()
    return (q - z).to(torch.float16) * s


# ----------------------------------------------------------------------------- ops


def linear(x: torch.Tensor, qweight_t: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor,
           bias: torch.Tensor | None, group_size: int, epilogue: str = "none",
           residual: torch.Tensor | None = None) -> torch.Tensor:
    """``x [M, K]`` fp16 times the dequantized weights in fp32, plus bias in fp32, rounded to
    fp16 once; then the epilogue as its unfused fp16 torch expression (``residual + y``, or
    ``silu(y[:, :N/2]) * y[:, N/2:]``)."""
    w = dequantize(qweight_t, scales, qzeros, group_size)
    acc = x.to(torch.float32) @ w.to(torch.float32).t()
    if bias is not None:
        acc = acc + bias.to(torch.float32)
    return _epilogue(acc.to(torch.float16), epilogue, residual)


def w4a8_linear(x8: torch.Tensor, x_scale: torch.Tensor, qweight_t: torch.Tensor, scales: torch.Tensor,
                qzeros: torch.Tensor, bias: torch.Tensor | None, group_size: int, epilogue: str = "none",
                residual: torch.Tensor | None = None) -> torch.Tensor:
    """``x_scale * (e4m3(x8) @ W^T) + bias`` in fp32 (W the fp16-dequantized weights), rounded
    to fp16 once; then the epilogue."""
    w = dequantize(qweight_t, scales, qzeros, group_size)
    acc = (x8.to(torch.float32) @ w.to(torch.float32).t()) * x_scale.to(torch.float32).reshape(-1, 1)
    if bias is not None:
        acc = acc + bias.to(torch.float32)
    return _epilogue(acc.to(torch.float16), epilogue, residual)


def _epilogue(y: torch.Tensor, epilogue: str, residual: torch.Tensor | None) -> torch.Tensor:
    if epilogue == "residual":
        assert residual is not None
        return residual + y
    if epilogue == "silu_mul":
        half = y.shape[-1] // 2
        return torch.nn.functional.silu(y[:, :half]) * y[:, half:]
    return y


def rmsnorm_fp8_quant(x: torch.Tensor, weight: torch.Tensor, eps: float,
                      scale: torch.Tensor | None) -> tuple[torch.Tensor, torch.Tensor]:
    """HF Qwen2 RMSNorm (fp32 mean of squares, ``x * rsqrt(ms + eps)`` rounded to fp16, then
    ``* weight`` in fp16), then e4m3 codes of ``y / scale`` clamped to ±448: per row with
    ``scale = max(amax(|y|) / 448, 1 / (448 * 512))``, or the given static scale."""
    xf = x.to(torch.float32)
    mean_sq = xf.pow(2).mean(dim=-1, keepdim=True)
    y = (xf * torch.rsqrt(mean_sq + eps)).to(x.dtype) * weight
    yf = y.to(torch.float32)
    if scale is None:
        s = (yf.abs().amax(dim=-1, keepdim=True) / FP8_E4M3_MAX).clamp(min=MIN_SCALE)
    else:
        s = scale
    q = (yf / s).clamp(-FP8_E4M3_MAX, FP8_E4M3_MAX).to(torch.float8_e4m3fn)
    return q, s


def rmsnorm_fp8_quant_dequant(x: torch.Tensor, weight: torch.Tensor, eps: float,
                              scale: torch.Tensor | None) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """:func:`rmsnorm_fp8_quant` plus ``(q.to(float32) * scale).to(float16)``."""
    q, s = rmsnorm_fp8_quant(x, weight, eps, scale)
    return q, s, (q.to(torch.float32) * s).to(torch.float16)
