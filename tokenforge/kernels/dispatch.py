"""Pure-Python kernel dispatch (dispatch.py:1-104 in the reference).

:func:`layer_support` is consulted when a layer's weights are loaded: it says whether this
path can serve the layer at all, and a layer it turns down stays with the caller's own linear
method (counted in ``tokenforge_fallback_total{reason}``). :func:`select` is consulted on every
call and looks only at M and the backend string. Since it never reads tensor contents, a
call through it can be captured into a HIP graph or traced by torch.compile.

There is one device path: hand-written HIP kernels for gfx950. ``backend`` keeps the
reference's string argument; ``"hip"`` is canonical and the reference's ``"triton"`` and
``"cuda"`` are accepted as aliases of the same path, so reference-shaped callers work
unchanged. ``"marlin"`` remains the per-layer kill switch.

:func:`select` takes the reference's keywords (``on_gpu``, ``triton_ok``,
``cuda_ext_available``) and returns the reference's decision for a call that cannot run on
the GPU: ``torch_reference``. For host tensors the ops follow it into the torch route
(``tokenforge.kernels.host``), as the reference does. For GPU tensors it means the kernel
library is missing or the GPU is not gfx950, and the ops raise :class:`HipUnavailableError`
naming the reason: a GPU call fails loudly instead of running a slow fallback.
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Final, Literal, get_args

from tokenforge.kernels.config import MAX_BUCKET_M, family_for_bucket, m_bucket
from tokenforge.kernels.device import SUPPORTED_ARCHS
from tokenforge.kernels.metrics import FALLBACKS, KERNEL_CALLS
from tokenforge.kernels.pack import PACK_FACTOR, SUPPORTED_GROUP_SIZES

Backend = Literal["hip", "triton", "cuda", "marlin"]
Kernel = Literal["hip_gemv", "hip_gemm", "torch_reference"]
FallbackReason = Literal[
    "kill_switch",
    "unsupported_dtype",
    "unsupported_group_size",
    "unsupported_shape",
    "unsupported_arch",
    "cuda_ext_unavailable",
]

BACKENDS: Final[tuple[str, ...]] = get_args(Backend)
HIP_BACKENDS: Final[tuple[str, ...]] = ("hip", "triton", "cuda")
BACKEND_ENV: Final = "TOKENFORGE_BACKEND"


class HipUnavailableError(RuntimeError):
    """The call cannot run on the HIP kernels and this build has no other path."""


def backend_from_env() -> Backend:
    value = os.environ.get(BACKEND_ENV, "hip").strip().lower()
    if value not in BACKENDS:
        raise ValueError(f"{BACKEND_ENV}={value!r} is not one of {BACKENDS}")
    return value  # type: ignore[return-value]


def layer_support(
    n: int, k: int, group_size: int, dtype: str, arch: str | None, backend: Backend
) -> FallbackReason | None:
    """``None`` if the HIP kernels can serve this layer, else the fallback reason.

    ``arch`` is the device's gfx architecture (``device.device_arch``), None when unknown.
    """
    if backend == "marlin":
        return "kill_switch"
    if dtype not in ("float16", "torch.float16"):
        return "unsupported_dtype"
    if group_size not in SUPPORTED_GROUP_SIZES:
        return "unsupported_group_size"
    if k % group_size != 0 or k % PACK_FACTOR != 0 or n % PACK_FACTOR != 0 or n <= 0:
        return "unsupported_shape"
    if arch is not None and arch not in SUPPORTED_ARCHS:
        return "unsupported_arch"
    return None


def record_layer_fallback(reason: FallbackReason) -> None:
    FALLBACKS.inc(reason=reason)


@dataclass(frozen=True)
class Decision:
    kernel: Kernel
    bucket: str
    fallback: FallbackReason | None = None


def bucket_label(m: int) -> str:
    return f">{MAX_BUCKET_M}" if m > MAX_BUCKET_M else str(m_bucket(m))


def lookup_bucket(m: int) -> int:
    """Autotune bucket of a call with ``m`` rows (M above the largest bucket uses it)."""
    return MAX_BUCKET_M if m > MAX_BUCKET_M else m_bucket(m)


def select(
    m: int,
    *,
    backend: Backend,
    on_gpu: bool,
    triton_ok: bool | None = None,
    cuda_ext_available: bool | None = None,
    hip_ok: bool | None = None,
) -> Decision:
    """Kernel family for one call with ``m`` rows. The layer has passed :func:`layer_support`.

    ``triton_ok`` (the reference's name) and ``hip_ok`` both mean "the compiled kernels can
    run this call" (library loaded, gfx950 device); either may be given, and an omitted flag
    counts as true. ``cuda_ext_available`` is accepted for the reference's signature: the one
    HIP library is this build's compiled extension, so it never splits the decision.
    """
    del cuda_ext_available
    if backend == "marlin":
        raise ValueError("backend 'marlin' is resolved per layer, not per call")
    bucket = bucket_label(m)
    runnable = (triton_ok is None or triton_ok) and (hip_ok is None or hip_ok)
    if not on_gpu or not runnable:
        return Decision("torch_reference", bucket)
    kernel: Kernel = "hip_gemv" if family_for_bucket(lookup_bucket(m)) == "gemv" else "hip_gemm"
    return Decision(kernel, bucket)


def require_gpu_decision(decision: Decision, *, on_gpu: bool) -> None:
    """Raise :class:`HipUnavailableError` for a ``torch_reference`` decision on a call the
    kernels must run (the ops send host tensors to the torch route before asking)."""
    if decision.kernel != "torch_reference":
        return
    if not on_gpu:
        raise HipUnavailableError(
            "this call needs GPU tensors; host tensors take the ops' torch route "
            "(tokenforge.kernels.host)"
        )
    raise HipUnavailableError(
        "the HIP kernel library is not loaded or the GPU is not gfx950 "
        "(build it with `python -m tokenforge_amd.build`)"
    )


def record(decision: Decision) -> None:
    KERNEL_CALLS.inc(kernel=decision.kernel, bucket=decision.bucket)
    if decision.fallback is not None:
        FALLBACKS.inc(reason=decision.fallback)
