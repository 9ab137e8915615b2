"""Helpers shared by the launchers: device checks, stream handle, device guard."""

from __future__ import annotations

import contextlib
from collections.abc import Iterator

import torch

from tokenforge_amd.kernels import _lib
from tokenforge_amd.kernels.device import SUPPORTED_ARCHS, device_arch


def require_gpu(name: str, *tensors: torch.Tensor) -> torch.device:
    """All tensors on one gfx950 device, library loaded; else raise (no CPU path)."""
    dev = tensors[0].device
    for t in tensors:
        if t.device != dev:
            raise ValueError(f"{name}: all tensors must be on one device, got {t.device} and {dev}")
    if dev.type != "cuda":
        raise RuntimeError(
            f"{name}: tokenforge_amd runs on gfx950 GPU tensors only, got a {dev.type} tensor "
            "(there is no CPU path)"
        )
    arch = device_arch(dev)
    if arch not in SUPPORTED_ARCHS:
        raise RuntimeError(f"{name}: device {dev} is {arch}, kernels are built for {SUPPORTED_ARCHS}")
    _lib.lib()  # raises HipLibraryError when the library is missing
    return dev


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
