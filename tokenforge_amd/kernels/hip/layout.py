"""Load-time int4 layout kernels on gfx950: pack, unpack, AWQ <-> TokenForge repack."""

from __future__ import annotations

import torch

from tokenforge_amd.kernels import _lib
from tokenforge_amd.kernels.hip._common import on_device, require_gpu, stream_of

PACK_FACTOR = 8


def pack_int4(values: torch.Tensor) -> torch.Tensor:
    """Pack 4-bit values along the last dim into int32 words, AWQ interleave (pack.py:42-54).

    Like the reference, values outside [0, 15] raise ``ValueError``; that check reads one
    device flag, so this load-time function synchronizes with the stream.
    """
    if values.shape[-1] % PACK_FACTOR != 0:
        raise ValueError(f"last dim {values.shape[-1]} is not a multiple of {PACK_FACTOR}")
    dev = require_gpu("pack_int4", values)
    *lead, n = values.shape
    v = values.to(torch.int32).contiguous()
    out = torch.empty((*lead, n // PACK_FACTOR), dtype=torch.int32, device=dev)
    if v.numel() == 0:
        return out
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    rows = v.numel() // n
    with on_device(dev):
        rc = _lib.lib().tf_pack_int4(v.data_ptr(), out.data_ptr(), rows, n, flag.data_ptr(), stream_of(dev))
    _lib.check(rc, "tf_pack_int4")
    if int(flag.item()) != 0:
        raise ValueError("int4 values must lie in [0, 15]")
    return out


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    """Inverse of :func:`pack_int4`. Returns int32 values in [0, 15] (pack.py:57-67)."""
    if packed.dtype != torch.int32:
        raise TypeError(f"packed tensor must be int32, got {packed.dtype}")
    dev = require_gpu("unpack_int4", packed)
    p = packed.contiguous()
    *lead, w = p.shape
    out = torch.empty((*lead, w * PACK_FACTOR), dtype=torch.int32, device=dev)
    if p.numel() == 0:
        return out
    with on_device(dev):
        rc = _lib.lib().tf_unpack_int4(p.data_ptr(), out.data_ptr(), p.numel() // w, w, stream_of(dev))
    _lib.check(rc, "tf_unpack_int4")
    return out


def _repack(src: torch.Tensor, forward: bool) -> torch.Tensor:
    if src.dtype != torch.int32:
        raise TypeError(f"packed tensor must be int32, got {src.dtype}")
    if src.dim() != 2:
        raise ValueError(f"packed weight must be 2-D, got shape {tuple(src.shape)}")
    dev = require_gpu("repack", src)
    s = src.contiguous()
    rows, words = s.shape
    cols = words * PACK_FACTOR
    if rows % PACK_FACTOR != 0:
        raise ValueError(f"{rows} rows is not a multiple of {PACK_FACTOR}")
    out = torch.empty((cols, rows // PACK_FACTOR), dtype=torch.int32, device=dev)
    if out.numel() == 0:
        return out
    h = _lib.lib()
    fn = h.tf_awq_to_tf if forward else h.tf_tf_to_awq
    with on_device(dev):
        rc = fn(s.data_ptr(), out.data_ptr(), rows, cols, stream_of(dev))
    _lib.check(rc, "repack")
    return out


def awq_to_tf(qweight: torch.Tensor) -> torch.Tensor:
    """AWQ ``qweight [K, N // 8]`` -> TokenForge ``qweight_t [N, K // 8]`` (pack.py:141-143)."""
    return _repack(qweight, forward=True)


def tf_to_awq(qweight_t: torch.Tensor) -> torch.Tensor:
    """Inverse of :func:`awq_to_tf` (pack.py:146-148)."""
    return _repack(qweight_t, forward=False)
