"""Helpers shared by the launchers: device checks, stream handle, device guard."""

from __future__ import annotations

import contextlib
from collections.abc import Iterator

import torch

from tokenforge.kernels import _lib
from tokenforge.kernels.device import SUPPORTED_ARCHS, device_arch


def require_gpu(name: str, *tensors: torch.Tensor) -> torch.device:
    """All tensors on one gfx950 device, library loaded; else raise (no CPU path)."""
    dev = tensors[0].device
    for t in tensors:
        if t.device != dev:
            raise ValueError(f"{name}: all tensors must be on one device, got {t.device} and {dev}")
    if dev.type != "cuda":
        raise RuntimeError(
            f"{name}: tokenforge.kernels runs on gfx950 GPU tensors only, got a {dev.type} tensor "
            "(there is no CPU path)"
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
    Per-call ops do not do this; they raise on host tensors. Without a visible GPU this raises:
    there is no CPU implementation.
    """
    home = tensors[0].device
    for t in tensors:
        if t.device != home:
            raise ValueError(f"{name}: all tensors must be on one device, got {t.device} and {home}")
    if home.type == "cuda":
        return home, home
    if not torch.cuda.is_available():
        raise RuntimeError(
            f"{name}: tokenforge.kernels runs on a gfx950 GPU; got {home.type} tensors and no GPU "
            "is visible (there is no CPU path)"
        )
    return torch.device("cuda", torch.cuda.current_device()), home


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
