"""Numpy restatement of the reference's numerics oracles (reference.py:1-56) and of the e4m3
rounding of rmsnorm_fp8.py:29-41.

Test infrastructure only (see ``oracle/__init__.py``).

One deliberate, documented difference: :func:`rmsnorm` forms the sum of squares in fp64 in
one fixed order (:func:`sum_squares`: every x^2 of an fp16 x is exact, the chunk sums and a
pairwise tree over the chunks round in fp64) and rounds it once to fp32, where reference.py:37
uses torch's fp32 ``mean``, whose own summation order can land one ulp away. Every HIP form
of the norm (the kernel's row per workgroup and row per wave, the decode GEMV's prologue) adds
in this same order, so kernel and oracle agree bit for bit whatever the batch size or fusion;
:func:`rmsnorm_torch_order` restates reference.py:37-39 with torch's own reduction for the
comparison against the reference as written.
"""

from __future__ import annotations

import numpy as np

from oracle.pack import W4A16Weights, dequantize_tf

FP8_E4M3_MAX = 448.0  # reference.py:9
MIN_SCALE = 1.0 / (FP8_E4M3_MAX * 512.0)  # reference.py:10
_F32_MIN_SCALE = np.float32(MIN_SCALE)
_F32_MAX = np.float32(FP8_E4M3_MAX)


def w4a16_reference(x: np.ndarray, weights: W4A16Weights, bias: np.ndarray | None = None) -> np.ndarray:
    """reference.py:13-21: fp64 ``x @ W^T (+ bias)`` on the fp16-dequantized weights.

    With non-finite inputs the product is formed elementwise, so inf * 0 -> NaN and
    inf - inf -> NaN exactly as IEEE arithmetic (a BLAS may skip zero operands).
    """
    w = dequantize_tf(weights).astype(np.float64)
    x64 = np.asarray(x).astype(np.float64)
    if np.isfinite(x64).all():
        y = x64 @ w.T
    else:
        y = (x64[:, None, :] * w[None, :, :]).sum(axis=-1)
    if bias is not None:
        y = y + np.asarray(bias).astype(np.float64)
    return y


def w4a16_fp32(x: np.ndarray, weights: W4A16Weights, bias: np.ndarray | None = None) -> np.ndarray:
    """reference.py:24-32: dequantize per call, fp32 matmul, (+ bias in fp32), cast to fp16.

    This is the reference's CPU path (ops.py:79-81), timed as the CPU baseline.
    """
    w = dequantize_tf(weights).astype(np.float32)
    y = np.asarray(x).astype(np.float32) @ w.T
    if bias is not None:
        y = y + np.asarray(bias).astype(np.float32)
    return y.astype(np.float16)


def sum_squares(x: np.ndarray) -> np.ndarray:
    """The row sums of x^2 (fp16 x, last axis) in fp64, in the norm's fixed order: elements in
    chunks of 8 (the row zero-padded to a multiple of 8), each chunk summed as
    ((e0 + e1) + (e2 + e3)) + ((e4 + e5) + (e6 + e7)) with e = fp64(x)^2 (exact), then the
    chunk sums added pairwise, bottom up over the chunk index: (c0 + c1), (c2 + c3), ..., then
    those pairs, and so on, the chunk count zero-padded to a power of two (adding zeros changes
    no partial sum). Returns [..., 1]."""
    x64 = np.asarray(x, dtype=np.float16).astype(np.float64)
    h = x64.shape[-1]
    pad = (-h) % 8
    if pad:
        x64 = np.concatenate([x64, np.zeros((*x64.shape[:-1], pad))], axis=-1)
    e = (x64 * x64).reshape(*x64.shape[:-1], -1, 8)
    pairs = e[..., 0::2] + e[..., 1::2]
    quads = pairs[..., 0::2] + pairs[..., 1::2]
    c = quads[..., 0] + quads[..., 1]
    n = c.shape[-1]
    width = 1
    while width < n:
        width *= 2
    if width > n:
        c = np.concatenate([c, np.zeros((*c.shape[:-1], width - n))], axis=-1)
    while c.shape[-1] > 1:
        c = c[..., 0::2] + c[..., 1::2]
    return c


def rmsnorm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """reference.py:35-39 (HF Qwen2 RMSNorm): fp32 normalize, round to fp16, times weight in
    fp16. The fp32 mean is the fixed-order fp64 sum (:func:`sum_squares`) rounded to fp32,
    divided by H (see module docstring)."""
    x16 = np.asarray(x, dtype=np.float16)
    h = x16.shape[-1]
    xf = x16.astype(np.float32)
    ss = sum_squares(x16)
    var = ss.astype(np.float32) / np.float32(h)
    rstd = np.float32(1.0) / np.sqrt(var + np.float32(eps))
    return (xf * rstd).astype(np.float16) * np.asarray(weight, dtype=np.float16)


def rmsnorm_torch_order(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """reference.py:35-39 with torch's own fp32 ``mean`` and ``rsqrt`` (library routines)."""
    import torch

    xt = torch.from_numpy(np.asarray(x, dtype=np.float16))
    wt = torch.from_numpy(np.asarray(weight, dtype=np.float16))
    xf = xt.to(torch.float32)
    var = xf.pow(2).mean(dim=-1, keepdim=True)
    return ((xf * torch.rsqrt(var + eps)).to(torch.float16) * wt).numpy()


def e4m3_encode(values: np.ndarray) -> np.ndarray:
    """Round fp32 values with |v| <= 448 (or NaN) to OCP e4m3fn codes, ties to even.

    Follows the rounding of rmsnorm_fp8.py:29-41 (normals keep 3 mantissa bits with RNE in
    fp32 bit space, subnormals use the fixed 2^-9 quantum, the sign is kept for +-0) and the
    e4m3fn format: bias 7, S.1111.111 = NaN. Returns uint8 codes.
    """
    v = np.asarray(values, dtype=np.float32)
    bits = v.view(np.uint32)
    sign = (bits >> np.uint32(24)) & np.uint32(0x80)
    a = bits & np.uint32(0x7FFFFFFF)
    is_nan = a > np.uint32(0x7F800000)
    is_sub = a < np.uint32(0x3C800000)
    with np.errstate(over="ignore", invalid="ignore"):
        sub = np.rint(a.view(np.float32) * np.float32(512.0)).astype(np.uint32)
        r = a + np.uint32(0x7FFFF) + ((a >> np.uint32(20)) & np.uint32(1))
        normal = (r >> np.uint32(20)) - np.uint32(120 << 3)
    code = np.where(is_nan, np.uint32(0x7F), np.where(is_sub, sub, normal)) & np.uint32(0x7F)
    return (code | sign).astype(np.uint8)


_E4M3_TABLE: np.ndarray | None = None


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """e4m3fn codes -> fp32 values from the format definition (NaN for S.1111.111)."""
    global _E4M3_TABLE
    if _E4M3_TABLE is None:
        table = np.zeros(256, dtype=np.float32)
        for c in range(256):
            s = -1.0 if c & 0x80 else 1.0
            e = (c >> 3) & 0xF
            m = c & 7
            if e == 0xF and m == 7:
                table[c] = np.nan
            elif e == 0:
                table[c] = s * m * 2.0**-9
            else:
                table[c] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
        _E4M3_TABLE = table
    return _E4M3_TABLE[np.asarray(codes, dtype=np.uint8)]


def w4a8_reference(
    codes: np.ndarray, x_scale: np.ndarray, weights: W4A16Weights, bias: np.ndarray | None = None
) -> np.ndarray:
    """W4A8 (no counterpart in the reference; the build's definition): fp64
    ``x_scale[m] * (e4m3(codes) @ W^T) (+ bias)``: :func:`w4a16_reference` (reference.py:13-21)
    on the decoded activations, times the row scale, before the bias. ``x_scale`` holds one
    scale or one per row."""
    x = e4m3_decode(codes).astype(np.float64)
    y = w4a16_reference(x, weights)
    s = np.asarray(x_scale, dtype=np.float64).reshape(-1)
    y = y * (s[:, None] if s.size > 1 else s[0])
    if bias is not None:
        y = y + np.asarray(bias).astype(np.float64)
    return y


def w4a8_exact_reference(
    codes: np.ndarray, x_scale: np.ndarray, weights: W4A16Weights, bias: np.ndarray | None = None
) -> np.ndarray:
    """W4A8 on exact weights (no counterpart in the reference; the build's definition for its
    fp8 GEMM): fp64 ``x_scale[m] * sum_g s[g][n] * sum_{k in g} e4m3(codes[m][k]) * (q - z)``
    (+ bias). Unlike :func:`w4a8_reference` the weights are not rounded to fp16: ``(q - z) * s``
    is exact in fp64 (a 5-bit integer times an fp16 scale). ``x_scale`` holds one scale or one
    per row."""
    from oracle.pack import unpack_int4

    g = weights.group_size
    q = unpack_int4(weights.qweight_t).astype(np.float64)  # [N, K]
    z = np.repeat(unpack_int4(weights.qzeros), g, axis=0).T.astype(np.float64)
    sc = np.repeat(np.asarray(weights.scales, dtype=np.float16), g, axis=0).T.astype(np.float64)
    w = (q - z) * sc
    x = e4m3_decode(codes).astype(np.float64)
    y = x @ w.T if np.isfinite(x).all() else (x[:, None, :] * w[None, :, :]).sum(axis=-1)
    s = np.asarray(x_scale, dtype=np.float64).reshape(-1)
    y = y * (s[:, None] if s.size > 1 else s[0])
    if bias is not None:
        y = y + np.asarray(bias).astype(np.float64)
    return y


def fp8_quant_reference(y: np.ndarray, scale: np.ndarray | None = None) -> tuple[np.ndarray, np.ndarray]:
    """reference.py:42-50: per-token dynamic (or static) saturating e4m3 quantization.

    Returns ``(codes uint8 [T, H], scale fp32 [T, 1] or the given static scale)``. NaN
    propagates through amax, the clamp and the cast like torch's ops.
    """
    yf = np.asarray(y).astype(np.float32)
    if scale is None:
        amax = np.max(np.abs(yf), axis=-1, keepdims=True)
        scale = np.maximum(amax / _F32_MAX, _F32_MIN_SCALE)
    else:
        scale = np.asarray(scale, dtype=np.float32)
    q = np.clip(yf / scale, -_F32_MAX, _F32_MAX)
    return e4m3_encode(q), scale.astype(np.float32)


def rmsnorm_fp8_reference(
    x: np.ndarray, weight: np.ndarray, eps: float, scale: np.ndarray | None = None
) -> tuple[np.ndarray, np.ndarray]:
    """reference.py:53-56."""
    return fp8_quant_reference(rmsnorm(x, weight, eps), scale)
