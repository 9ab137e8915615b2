"""Device identity helpers (device.py:1-35 in the reference), keyed on the gfx architecture.

On ROCm, ``torch.cuda.get_device_capability`` reports a CUDA-style pair (9, 5 on MI355X),
which would produce a misleading ``sm95`` slug; the architecture name ``gfx950`` from
``gcnArchName`` is the stable key here. None of these read tensor values or synchronize.
"""

from __future__ import annotations

import functools
import re

import torch

from tokenforge.kernels import _lib

SUPPORTED_ARCHS: tuple[str, ...] = ("gfx950",)


@functools.cache
def _arch_of_index(index: int) -> str:
    name = torch.cuda.get_device_properties(index).gcnArchName
    return name.split(":")[0]


def device_arch(device: torch.device) -> str | None:
    """``gfx950`` for an MI355X, None off-GPU."""
    if device.type != "cuda":
        return None
    index = device.index if device.index is not None else torch.cuda.current_device()
    return _arch_of_index(index)


def hip_runnable(t: torch.Tensor) -> bool:
    """Whether the HIP kernels can run on this tensor in the current process."""
    return t.is_cuda and device_arch(t.device) in SUPPORTED_ARCHS and _lib.available()


def gpu_identity(device: torch.device) -> str:
    """Stable, filesystem-safe id of the device, e.g. ``amd-gfx950-256cu`` for an MI355X.

    Built from the architecture and the compute-unit count, which identify the kernel
    tuning target. The marketing name is not used: ROCm reports it inconsistently (an
    empty string under some profilers, a generic "AMD Radeon Graphics" elsewhere).
    """
    if device.type != "cuda":
        return "cpu"
    index = device.index if device.index is not None else torch.cuda.current_device()
    cus = torch.cuda.get_device_properties(index).multi_processor_count
    arch = re.sub(r"[^a-z0-9]+", "-", str(device_arch(device)).lower()).strip("-")
    return f"amd-{arch}-{cus}cu"
