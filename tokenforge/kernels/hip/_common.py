"""Helpers shared by the launchers: device checks, stream handle, device guard."""

from __future__ import annotations

import contextlib
from collections.abc import Iterator

import torch

from tokenforge.kernels import _lib
from tokenforge.kernels.device import SUPPORTED_ARCHS, device_arch


def require_gpu(name: str, *tensors: torch.Tensor) -> torch.device:
    """All tensors on one gfx950 device, library loaded; else raise. These are the kernel
    launchers: host tensors reach them only by mistake (the ops send them to the torch route)."""
    dev = tensors[0].device
    for t in tensors:
        if t.device != dev:
            raise ValueError(f"{name}: all tensors must be on one device, got {t.device} and {dev}")
    if dev.type != "cuda":
        raise RuntimeError(
            f"{name}: the HIP kernels take gfx950 GPU tensors, got a {dev.type} tensor "
            "(the ops in torch.ops.tokenforge take host tensors through their torch route)"
        )
    arch = device_arch(dev)
    if arch not in SUPPORTED_ARCHS:
        raise RuntimeError(f"{name}: device {dev} is {arch}, kernels are built for {SUPPORTED_ARCHS}")
    _lib.lib()  # raises HipLibraryError when the library is missing
    return dev


def load_time_devices(name: str, *tensors: torch.Tensor) -> tuple[torch.device, torch.device]:
    """(device to run on, device to return results on) for a load-time function.

    Load-time functions (packing, repacking, quantizing fixtures) accept host tensors like
    the reference's: their inputs are copied to the current GPU and the results copied back.
    Per-call ops do not do this; they send host tensors to the torch route. Without a visible
    GPU the load-time functions take the torch route too (:func:`host_route`), before this.
    """
    home = tensors[0].device
    for t in tensors:
        if t.device != home:
            raise ValueError(f"{name}: all tensors must be on one device, got {t.device} and {home}")
    if home.type == "cuda":
        return home, home
    if not torch.cuda.is_available():
        raise RuntimeError(
            f"{name}: got {home.type} tensors, which run on a gfx950 GPU or (host tensors, no GPU "
            "visible) the torch route"
        )
    return torch.device("cuda", torch.cuda.current_device()), home


def host_route(*tensors: torch.Tensor) -> bool:
    """Whether a load-time function takes the torch route (``tokenforge.kernels.host``): every
    tensor is on the host and no GPU is visible. With a GPU visible, host tensors go to it."""
    return all(t.device.type == "cpu" for t in tensors) and not torch.cuda.is_available()


def stream_of(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


@contextlib.contextmanager
def on_device(dev: torch.device) -> Iterator[None]:
    """Make ``dev`` current for the launch when it is not already."""
    if dev.index is None or dev.index == torch.cuda.current_device():
        yield
        return
    with torch.cuda.device(dev):
        yield


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
