"""Load-time int4 layout kernels on gfx950: pack, unpack, AWQ <-> TokenForge repack, the tile
layout permutation and the AWQ fixture quantizer.

These run at weight-load time. They accept host tensors too (see
``_common.load_time_devices``): the kernel runs on the current GPU and the result comes back on
the input's device. With no GPU visible, host tensors take the torch route
(``tokenforge.kernels.host``), which produces the same bits.
"""

from __future__ import annotations

import torch

from tokenforge.kernels import _lib, host
from tokenforge.kernels.hip._common import host_route, load_time_devices, on_device, require_gpu, stream_of

PACK_FACTOR = 8


def pack_int4(values: torch.Tensor) -> torch.Tensor:
    """Pack 4-bit values along the last dim into int32 words, AWQ interleave (pack.py:42-54).

    Like the reference, values outside [0, 15] raise ``ValueError``; that check reads one
    device flag, so this load-time function synchronizes with the stream.
    """
    if values.shape[-1] % PACK_FACTOR != 0:
        raise ValueError(f"last dim {values.shape[-1]} is not a multiple of {PACK_FACTOR}")
    if host_route(values):
        return host.pack_int4(values)
    run, home = load_time_devices("pack_int4", values)
    dev = require_gpu("pack_int4", values.to(run))
    *lead, n = values.shape
    v = values.to(device=dev, dtype=torch.int32).contiguous()
    out = torch.empty((*lead, n // PACK_FACTOR), dtype=torch.int32, device=dev)
    if v.numel() == 0:
        return out.to(home)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    rows = v.numel() // n
    with on_device(dev):
        rc = _lib.lib().tf_pack_int4(v.data_ptr(), out.data_ptr(), rows, n, flag.data_ptr(), stream_of(dev))
    _lib.check(rc, "tf_pack_int4")
    if int(flag.item()) != 0:
        raise ValueError("int4 values must lie in [0, 15]")
    return out.to(home)


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    """Inverse of :func:`pack_int4`. Returns int32 values in [0, 15] (pack.py:57-67)."""
    if packed.dtype != torch.int32:
        raise TypeError(f"packed tensor must be int32, got {packed.dtype}")
    if host_route(packed):
        return host.unpack_int4(packed)
    run, home = load_time_devices("unpack_int4", packed)
    p = packed.to(run).contiguous()
    dev = require_gpu("unpack_int4", p)
    *lead, w = p.shape
    out = torch.empty((*lead, w * PACK_FACTOR), dtype=torch.int32, device=dev)
    if p.numel() == 0:
        return out.to(home)
    with on_device(dev):
        rc = _lib.lib().tf_unpack_int4(p.data_ptr(), out.data_ptr(), p.numel() // w, w, stream_of(dev))
    _lib.check(rc, "tf_unpack_int4")
    return out.to(home)


def _repack(src: torch.Tensor, forward: bool) -> torch.Tensor:
    if src.dtype != torch.int32:
        raise TypeError(f"packed tensor must be int32, got {src.dtype}")
    if src.dim() != 2:
        raise ValueError(f"packed weight must be 2-D, got shape {tuple(src.shape)}")
    if host_route(src):
        return host.transpose_packed(src)
    run, home = load_time_devices("repack", src)
    s = src.to(run).contiguous()
    dev = require_gpu("repack", s)
    rows, words = s.shape
    cols = words * PACK_FACTOR
    if rows % PACK_FACTOR != 0:
        raise ValueError(f"{rows} rows is not a multiple of {PACK_FACTOR}")
    out = torch.empty((cols, rows // PACK_FACTOR), dtype=torch.int32, device=dev)
    if out.numel() == 0:
        return out.to(home)
    h = _lib.lib()
    fn = h.tf_awq_to_tf if forward else h.tf_tf_to_awq
    with on_device(dev):
        rc = fn(s.data_ptr(), out.data_ptr(), rows, cols, stream_of(dev))
    _lib.check(rc, "repack")
    return out.to(home)


def awq_to_tf(qweight: torch.Tensor) -> torch.Tensor:
    """AWQ ``qweight [K, N // 8]`` -> TokenForge ``qweight_t [N, K // 8]`` (pack.py:141-143)."""
    return _repack(qweight, forward=True)


def tf_to_awq(qweight_t: torch.Tensor) -> torch.Tensor:
    """Inverse of :func:`awq_to_tf` (pack.py:146-148)."""
    return _repack(qweight_t, forward=False)


def _tile(qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor, group_size: int,
          to_tile: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    name = "tile_pack" if to_tile else "tile_unpack"
    if qweight.dtype != torch.int32 or qzeros.dtype != torch.int32:
        raise TypeError(f"{name}: qweight and qzeros must be int32")
    if scales.dtype != torch.float16:
        raise TypeError(f"{name}: scales must be fp16, got {scales.dtype}")
    if qweight.dim() != 2:
        raise ValueError(f"{name}: qweight must be 2-D [N, K/8], got shape {tuple(qweight.shape)}")
    n, k = qweight.shape[0], qweight.shape[1] * PACK_FACTOR
    if group_size <= 0 or k % group_size:
        raise ValueError(f"{name}: K={k} is not a multiple of group_size={group_size}")
    if tuple(scales.shape) != (k // group_size, n):
        raise ValueError(f"{name}: scales shape {tuple(scales.shape)} != {(k // group_size, n)}")
    if tuple(qzeros.shape) != (k // group_size, n // PACK_FACTOR):
        raise ValueError(f"{name}: qzeros shape {tuple(qzeros.shape)} != {(k // group_size, n // PACK_FACTOR)}")
    if host_route(qweight, scales, qzeros):
        return (host.tile_pack if to_tile else host.tile_unpack)(qweight, scales, qzeros, group_size)
    run, home = load_time_devices(name, qweight, scales, qzeros)
    qw, sc, qz = (t.to(run).contiguous() for t in (qweight, scales, qzeros))
    dev = require_gpu(name, qw, sc, qz)
    outs = tuple(torch.empty_like(t) for t in (qw, sc, qz))
    if qw.numel() == 0:
        return tuple(o.to(home) for o in outs)  # type: ignore[return-value]
    fn = _lib.lib().tf_tile_pack if to_tile else _lib.lib().tf_tile_unpack
    with on_device(dev):
        rc = fn(qw.data_ptr(), sc.data_ptr(), qz.data_ptr(), outs[0].data_ptr(), outs[1].data_ptr(),
                outs[2].data_ptr(), n, k, group_size, stream_of(dev))
    _lib.check(rc, name)
    return tuple(o.to(home) for o in outs)  # type: ignore[return-value]


def tile_pack(qweight_t: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor,
              group_size: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """TokenForge-layout ``(qweight_t, scales, qzeros)`` -> the gfx950 tile layout (same shapes)."""
    return _tile(qweight_t, scales, qzeros, group_size, to_tile=True)


def tile_unpack(qweight_t: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor,
                group_size: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Inverse of :func:`tile_pack`."""
    return _tile(qweight_t, scales, qzeros, group_size, to_tile=False)


def awq_quantize(weight: torch.Tensor, group_size: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Min-max asymmetric int4 of ``weight [N, K]`` into AWQ format (pack.py:83-107) on the GPU.

    Arithmetic in fp32 with IEEE division and round-half-to-even, as the reference's torch
    expression; weights must be finite."""
    if weight.dim() != 2:
        raise ValueError(f"weight must be 2-D [N, K], got shape {tuple(weight.shape)}")
    n, k = weight.shape
    if k % group_size != 0:
        raise ValueError(f"K={k} is not a multiple of group_size={group_size}")
    if n % PACK_FACTOR != 0:
        raise ValueError(f"N={n} is not a multiple of {PACK_FACTOR}")
    if host_route(weight):
        return host.awq_quantize(weight, group_size)
    run, home = load_time_devices("awq_quantize", weight)
    w = weight.to(device=run, dtype=torch.float32).contiguous()
    dev = require_gpu("awq_quantize", w)
    qweight = torch.empty((k, n // PACK_FACTOR), dtype=torch.int32, device=dev)
    qzeros = torch.empty((k // group_size, n // PACK_FACTOR), dtype=torch.int32, device=dev)
    scales = torch.empty((k // group_size, n), dtype=torch.float16, device=dev)
    if w.numel():
        with on_device(dev):
            rc = _lib.lib().tf_awq_quantize(w.data_ptr(), n, k, group_size, qweight.data_ptr(),
                                            qzeros.data_ptr(), scales.data_ptr(), stream_of(dev))
        _lib.check(rc, "tf_awq_quantize")
    return qweight.to(home), qzeros.to(home), scales.to(home)
