"""The TokenForge operators (ops.py:1-156 in the reference) on the gfx950 kernels.

The operators are registered with the PyTorch dispatcher by the C++ extension
``tokenforge_amd/lib/libtokenforge_torch.so`` (source ``tokenforge_amd/ext/torch_ops.cpp``),
loaded here: it defines the schemas and the GPU kernels, whose launch path is C++ (checks,
cached launch config, dispatch counter, one C-ABI call), a few microseconds of host time per
call. This module registers the rest: a fake (meta) implementation per operator, so
torch.compile traces each as one opaque node and HIP graphs capture it like any other launch;
the torch route for host tensors; the launch-config resolver the C++ side asks once per
(operator, epilogue, M, N, K, group size, device); and each operator's Python body
(``tokenforge::_py_<op>``), which the C++ kernel hands every call it does not launch itself
(bad arguments, empty inputs, tensors that need a copy) and which raises the reference's
exceptions or launches the same kernels. The real implementations never read tensor values on
the host and never synchronize.

Ops (same names and schemas as the reference):

* ``tokenforge::w4a16_linear(x, qweight_t, scales, qzeros, bias, group_size, backend)``
* ``tokenforge::w4a16_dequant(qweight_t, scales, qzeros, group_size)``
* ``tokenforge::rmsnorm_fp8_quant(x, weight, eps, scale)``

and two fused forms of the linear with no counterpart in the reference (which runs the same
arithmetic as separate torch ops after ``w4a16_linear``):

* ``tokenforge::w4a16_linear_residual(x, qweight_t, scales, qzeros, bias, residual, group_size,
  backend)`` = ``residual + w4a16_linear(...)``
* ``tokenforge::w4a16_linear_silu_mul(x, qweight_t, scales, qzeros, bias, group_size, backend)``
  = ``silu(y[..., :N/2]) * y[..., N/2:]`` with ``y = w4a16_linear(...)``

Each equals its unfused torch expression on fp16 tensors bit for bit (same roundings). And
the W4A8 form, which takes ``rmsnorm_fp8_quant``'s output directly (no counterpart either):

* ``tokenforge::w4a8_linear(x8, x_scale, qweight_t, scales, qzeros, bias, group_size, backend,
  epilogue, residual)`` = ``x_scale * (e4m3(x8) @ W^T) + bias`` (then the epilogue)

and the norm with the fp16 activation a W4A16 linear reads from its codes (no counterpart):

* ``tokenforge::rmsnorm_fp8_quant_dequant(x, weight, eps, scale)`` = ``(q, scale, a)`` with
  ``(q, scale) = rmsnorm_fp8_quant(...)`` and ``a = (q.to(float32) * scale).to(float16)``

and the decode norm-then-linear in one launch (no counterpart either):

* ``tokenforge::rmsnorm_fp8_w4a16_linear(x, norm_weight, eps, qweight_t, scales, qzeros, bias,
  group_size, backend, epilogue)`` = ``w4a16_linear(a, ...)`` (or its SiLU*mul form) with ``a``
  from ``rmsnorm_fp8_quant_dequant(x, norm_weight, eps, None)``; one kernel where the bucket's
  config is the GEMV stream form (M <= 4), the two kernels otherwise; same bits either way.

On GPU tensors every op runs the hand-written HIP kernels, and a missing kernel library (or
a GPU other than gfx950) raises instead of falling back. Host (CPU) tensors take the
reference's ``torch_reference`` route (ops.py:79-81): the torch expressions of
``tokenforge.kernels.host``, the same arithmetic the reference runs on the host.
"""

from __future__ import annotations

import ctypes
import dataclasses
import functools

import torch

from tokenforge.kernels import _lib, autotune, dispatch, host
from tokenforge.kernels.config import (
    M_BUCKETS,
    MAX_BUCKET_M,
    NUM_CUS,
    GemmConfig,
    fp8_gemm_applies,
    fp8_gemm_config,
    norm_fused_config,
    split_k_gemv_config,
    stream_form_applies,
)
from tokenforge.kernels.device import SUPPORTED_ARCHS, device_arch, gpu_identity
from tokenforge.kernels.hip import rmsnorm_fp8 as _rms
from tokenforge.kernels.hip import w4a16 as _w4a16
from tokenforge.kernels.metrics import KERNEL_CALLS


def _load_extension() -> None:
    """Load the operator extension (schemas and GPU kernels) and bind it to the kernel library
    this process uses; a missing extension raises here, at import."""
    path = _lib.torch_ops_path()
    if not path.exists():
        raise _lib.HipLibraryError(f"{path} is missing: build it with `python -m tokenforge_amd.build`")
    torch.ops.load_library(str(path))
    if _lib.available():
        torch.ops.tokenforge._bind_library(str(_lib.library_path()))


_load_extension()
_LIB = torch.library.Library("tokenforge", "FRAGMENT")


@functools.cache
def _gpu_id(device: torch.device) -> str:
    return gpu_identity(device)


def _on_host(op: str, *tensors: torch.Tensor | None) -> bool:
    """Whether a call takes the torch route: its tensors are host tensors. A call that mixes
    host and GPU tensors raises."""
    on_host = [t.device.type == "cpu" for t in tensors if t is not None]
    if not any(on_host):
        return False
    if not all(on_host):
        raise ValueError(f"{op}: all tensors must be on one device (got host and GPU tensors)")
    return True


def _record_host(m: int, backend: str) -> None:
    """The reference's decision for a host call (``torch_reference``), counted like any other."""
    dispatch.record(dispatch.select(m, backend=backend, on_gpu=False))  # type: ignore[arg-type]


def _gpu_config(device: torch.device, m: int, n: int, k: int, group_size: int) -> GemmConfig:
    """The launch config of a call with M rows on ``device`` (after the device check).

    A ``torch_reference`` decision here (library missing, other GPU) raises: GPU tensors never
    fall back. The tuned config may pick the other kernel family in the buckets both serve.
    """
    runnable = device_arch(device) in SUPPORTED_ARCHS and _lib.available()
    decision = dispatch.select(m, backend="hip", on_gpu=True, triton_ok=runnable,
                               cuda_ext_available=_lib.available())
    dispatch.require_gpu_decision(decision, on_gpu=True)
    cfg = autotune.lookup(_gpu_id(device), dispatch.lookup_bucket(m), n, k, group_size)
    if m > MAX_BUCKET_M and cfg.split_k > 1 and -(-m // cfg.block_m) * -(-n // cfg.block_n) >= NUM_CUS:
        # Above the largest bucket its config is reused; once the M tiles alone fill the CUs a
        # K split only adds the fp32 workspace (split * M * N * 4 bytes) and its reduction.
        cfg = dataclasses.replace(cfg, split_k=1)
    if cfg.stream and not stream_form_applies(m, n, k, cfg.num_warps, max_m=cfg.block_m, split_k=cfg.split_k):
        # The bucket's config is the stream form but this call is outside it (N % 32 == 16, or
        # an x too long to stage): the K-split GEMV runs it, whatever the epilogue.
        cfg = split_k_gemv_config(n, k)
    return cfg


def _family(cfg: GemmConfig) -> dispatch.Kernel:
    return "hip_gemm" if cfg.family == "gemm" else "hip_gemv"


def _decide(x2: torch.Tensor, m: int, n: int, k: int, group_size: int, backend: str) -> GemmConfig:
    """Dispatch decision and launch config of a call on GPU tensors (the Python body's path);
    the counter records the family that runs."""
    cfg = _gpu_config(x2.device, m, n, k, group_size)
    dispatch.record(dispatch.Decision(_family(cfg), dispatch.bucket_label(m)))
    return cfg


def _w4a8_config(cfg: GemmConfig, m: int, n: int, k: int, group_size: int) -> GemmConfig:
    """The W4A8 launch: at prefill M the e4m3 codes go straight into the fp8 MFMA (weights as
    exact e4m3 (q - z), the group scale applied in fp32) instead of being decoded to fp16."""
    bucket = dispatch.lookup_bucket(m)
    if cfg.family == "gemm" and fp8_gemm_applies(bucket, n, k, group_size):
        cfg = fp8_gemm_config(bucket, n, k)
        if m > MAX_BUCKET_M and cfg.split_k > 1 and -(-m // cfg.block_m) * -(-n // cfg.block_n) >= NUM_CUS:
            # As in _gpu_config: past the largest bucket, once the M tiles fill the CUs a K
            # split only adds its fp32 workspace and reduction.
            cfg = dataclasses.replace(cfg, split_k=1)
    return cfg


# ----------------------------------------------------------------------------- the C++ side's hooks

KIND_LINEAR, KIND_W4A8, KIND_NORM_LINEAR = 0, 1, 2
_EPILOGUE_NAMES = {_lib.EPILOGUE_NONE: "none", _lib.EPILOGUE_RESIDUAL: "residual", _lib.EPILOGUE_SILU_MUL: "silu_mul"}
_FAMILIES: tuple[dispatch.Kernel, ...] = ("hip_gemv", "hip_gemm")
_BUCKET_LABELS = tuple(str(b) for b in M_BUCKETS) + (f">{MAX_BUCKET_M}",)
_NATIVE_BUCKETS = 64  # the C++ counter table's bucket dimension


def _resolve_launch(kind: int, epilogue: int, m: int, n: int, k: int, group_size: int, device: int) -> list[int]:
    """The launch the C++ kernel makes for (kind, epilogue, M, N, K, group size, device):
    the config fields, the counter's family and bucket indices, the workspace bytes and, for
    the norm + linear, whether the GEMV's prologue runs the norm."""
    dev = torch.device("cuda", device)
    cfg = _gpu_config(dev, m, n, k, group_size)
    family = _FAMILIES.index(_family(cfg))
    fused = 0
    h = _lib.lib()
    if kind == KIND_W4A8:
        cfg = _w4a8_config(cfg, m, n, k, group_size)
        c = _w4a16.to_c_config(cfg)
        need = int(h.tf_w4a8_workspace_bytes_ex(m, n, k, group_size, ctypes.byref(c), epilogue))
    else:
        if kind == KIND_NORM_LINEAR:
            fcfg = norm_fused_config(cfg, m, n, k)
            if fcfg is not None:
                cfg, fused = fcfg, 1
        c = _w4a16.to_c_config(cfg)
        need = 0 if fused else int(h.tf_w4a16_workspace_bytes_ex(m, n, k, group_size, ctypes.byref(c), epilogue))
    bucket = _BUCKET_LABELS.index(dispatch.bucket_label(m))
    return [c.kernel, c.block_m, c.block_n, c.block_k, c.split_k, c.num_warps, c.num_stages, family, bucket, need,
            fused]


_LIB.impl("_resolve_launch", _resolve_launch, "CompositeExplicitAutograd")
autotune.on_change(torch.ops.tokenforge._clear_launch_cache)

_native_seen = [0] * (len(_FAMILIES) * _NATIVE_BUCKETS)


def _fold_native_calls() -> None:
    """Add the C++ kernels' dispatch counts since the last fold to ``KERNEL_CALLS``."""
    counts = torch.ops.tokenforge._native_calls()
    for i, c in enumerate(counts):
        delta = c - _native_seen[i]
        if delta:
            _native_seen[i] = c
            KERNEL_CALLS.inc(delta, kernel=_FAMILIES[i // _NATIVE_BUCKETS], bucket=_BUCKET_LABELS[i % _NATIVE_BUCKETS])


KERNEL_CALLS.set_pre_read(_fold_native_calls)


def _check_backend(backend: str) -> None:
    if backend not in dispatch.HIP_BACKENDS:
        raise ValueError(
            f"backend must be 'hip' (or its aliases 'triton', 'cuda') at op level, got {backend!r}"
        )


# ----------------------------------------------------------------------------- W4A16 linear


def _linear(
    x: torch.Tensor,
    qweight_t: torch.Tensor,
    scales: torch.Tensor,
    qzeros: torch.Tensor,
    bias: torch.Tensor | None,
    group_size: int,
    backend: str,
    epilogue: str = "none",
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    k = x.shape[-1]
    n = qweight_t.shape[0]
    n_out = n // 2 if epilogue == "silu_mul" else n
    out_shape = (*x.shape[:-1], n_out)
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    m = x2.shape[0]
    if m == 0:
        return x.new_empty(out_shape)
    _check_backend(backend)
    r2 = None
    if residual is not None:
        if tuple(residual.shape) != (*x.shape[:-1], n):
            raise ValueError(f"residual shape {tuple(residual.shape)} != {(*x.shape[:-1], n)}")
        r2 = residual.reshape(-1, n)
    if _on_host("w4a16_linear", x2, qweight_t, scales, qzeros, bias, r2):
        _, _, _, bias, r2 = _w4a16.check_linear_args(x2, qweight_t, scales, qzeros, group_size, bias, epilogue, r2)
        _record_host(m, backend)
        return host.linear(x2, qweight_t, scales, qzeros, bias, group_size, epilogue, r2).reshape(out_shape)
    cfg = _decide(x2, m, n, k, group_size, backend)
    y = _w4a16.w4a16_gemm_ex(x2, qweight_t, scales, qzeros, group_size, cfg, bias, epilogue, r2)
    return y.reshape(out_shape)


def _w4a16_linear(x, qweight_t, scales, qzeros, bias, group_size, backend):  # type: ignore[no-untyped-def]
    return _linear(x, qweight_t, scales, qzeros, bias, group_size, backend)


def _w4a16_linear_residual(x, qweight_t, scales, qzeros, bias, residual, group_size, backend):  # type: ignore[no-untyped-def]
    return _linear(x, qweight_t, scales, qzeros, bias, group_size, backend, "residual", residual)


def _w4a16_linear_silu_mul(x, qweight_t, scales, qzeros, bias, group_size, backend):  # type: ignore[no-untyped-def]
    return _linear(x, qweight_t, scales, qzeros, bias, group_size, backend, "silu_mul")


@torch.library.register_fake("tokenforge::w4a16_linear")
def _w4a16_linear_fake(x, qweight_t, scales, qzeros, bias, group_size, backend):  # type: ignore[no-untyped-def]
    return x.new_empty((*x.shape[:-1], qweight_t.shape[0]))


@torch.library.register_fake("tokenforge::w4a16_linear_residual")
def _w4a16_linear_residual_fake(x, qweight_t, scales, qzeros, bias, residual, group_size, backend):  # type: ignore[no-untyped-def]
    return x.new_empty((*x.shape[:-1], qweight_t.shape[0]))


@torch.library.register_fake("tokenforge::w4a16_linear_silu_mul")
def _w4a16_linear_silu_mul_fake(x, qweight_t, scales, qzeros, bias, group_size, backend):  # type: ignore[no-untyped-def]
    return x.new_empty((*x.shape[:-1], qweight_t.shape[0] // 2))


# ----------------------------------------------------------------------------- W4A8 linear


def _w4a8_linear(x8, x_scale, qweight_t, scales, qzeros, bias, group_size, backend, epilogue="none",  # type: ignore[no-untyped-def]
                 residual=None):
    """W4A8 linear on FP8 activations: ``x_scale * (e4m3(x8) @ dequant(W)^T) + bias`` with an
    optional epilogue ("none", "residual", "silu_mul"); ``x8``/``x_scale`` as
    ``rmsnorm_fp8_quant`` returns them (scale [..., 1] per row, or one static scale)."""
    k = x8.shape[-1]
    n = qweight_t.shape[0]
    n_out = n // 2 if epilogue == "silu_mul" else n
    out_shape = (*x8.shape[:-1], n_out)
    x2 = x8.reshape(-1, k)
    m = x2.shape[0]
    if m == 0:
        return x8.new_empty(out_shape, dtype=torch.float16)
    _check_backend(backend)
    if _on_host("w4a8_linear", x2, x_scale, qweight_t, scales, qzeros, bias, residual):
        r2 = residual.reshape(-1, n) if residual is not None else None
        _, _, _, bias, r2 = _w4a16.check_w4a8_args(x2, x_scale, qweight_t, scales, qzeros, group_size, bias,
                                                   epilogue, r2)
        _record_host(m, backend)
        y = host.w4a8_linear(x2, x_scale.reshape(-1), qweight_t, scales, qzeros, bias, group_size, epilogue, r2)
        return y.reshape(out_shape)
    cfg = _w4a8_config(_decide(x2, m, n, k, group_size, backend), m, n, k, group_size)
    # One contiguous scale vector: the kernel reads its data pointer with the stride of this view.
    s2 = (x_scale.reshape(-1) if x_scale.numel() > 1 else x_scale.reshape(1)).contiguous()
    r2 = residual.reshape(-1, n) if residual is not None else None
    y = _w4a16.w4a8_gemm_ex(x2, s2, qweight_t, scales, qzeros, group_size, cfg, bias, epilogue, r2)
    return y.reshape(out_shape)


@torch.library.register_fake("tokenforge::w4a8_linear")
def _w4a8_linear_fake(x8, x_scale, qweight_t, scales, qzeros, bias, group_size, backend, epilogue="none",  # type: ignore[no-untyped-def]
                      residual=None):
    n = qweight_t.shape[0]
    return x8.new_empty((*x8.shape[:-1], n // 2 if epilogue == "silu_mul" else n), dtype=torch.float16)


# ----------------------------------------------------------------------------- dequant


def _w4a16_dequant(qweight_t, scales, qzeros, group_size):  # type: ignore[no-untyped-def]
    if _on_host("w4a16_dequant", qweight_t, scales, qzeros):
        _w4a16.check_dequant_inputs(qweight_t, scales, qzeros, group_size)
        return host.dequantize(qweight_t, scales, qzeros, group_size)
    return _w4a16.w4a16_dequant(qweight_t, scales, qzeros, group_size)


@torch.library.register_fake("tokenforge::w4a16_dequant")
def _w4a16_dequant_fake(qweight_t, scales, qzeros, group_size):  # type: ignore[no-untyped-def]
    return qweight_t.new_empty((qweight_t.shape[0], qweight_t.shape[1] * 8), dtype=torch.float16)


# ----------------------------------------------------------------------------- RMSNorm + FP8


def _rmsnorm_fp8_quant(x, weight, eps, scale):  # type: ignore[no-untyped-def]
    h = x.shape[-1]
    x2 = x.reshape(-1, h)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    if _on_host("rmsnorm_fp8_quant", x2, weight, scale):
        _rms.check_inputs(x2, weight, scale)
        q, s = host.rmsnorm_fp8_quant(x2, weight, eps, scale)
    else:
        q, s = _rms.rmsnorm_fp8_quant(x2, weight, eps, scale)
    if scale is not None:
        s = s.clone()  # custom ops may not return an alias of an input
    return q.reshape(x.shape), s.reshape((*x.shape[:-1], 1)) if scale is None else s


@torch.library.register_fake("tokenforge::rmsnorm_fp8_quant")
def _rmsnorm_fp8_quant_fake(x, weight, eps, scale):  # type: ignore[no-untyped-def]
    q = x.new_empty(x.shape, dtype=torch.float8_e4m3fn)
    if scale is None:
        return q, x.new_empty((*x.shape[:-1], 1), dtype=torch.float32)
    return q, torch.empty_like(scale)


def _rmsnorm_fp8_quant_dequant(x, weight, eps, scale):  # type: ignore[no-untyped-def]
    """``rmsnorm_fp8_quant`` plus ``(q.to(float32) * scale).to(float16)`` from one launch (no
    counterpart in the reference): the fp16 activation of a W4A16 linear fed from the codes."""
    h = x.shape[-1]
    x2 = x.reshape(-1, h)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    if _on_host("rmsnorm_fp8_quant_dequant", x2, weight, scale):
        _rms.check_inputs(x2, weight, scale)
        q, s, a = host.rmsnorm_fp8_quant_dequant(x2, weight, eps, scale)
    else:
        q, s, a = _rms.rmsnorm_fp8_quant_dequant(x2, weight, eps, scale)
    if scale is not None:
        s = s.clone()  # custom ops may not return an alias of an input
    return q.reshape(x.shape), s.reshape((*x.shape[:-1], 1)) if scale is None else s, a.reshape(x.shape)


@torch.library.register_fake("tokenforge::rmsnorm_fp8_quant_dequant")
def _rmsnorm_fp8_quant_dequant_fake(x, weight, eps, scale):  # type: ignore[no-untyped-def]
    q, s = _rmsnorm_fp8_quant_fake(x, weight, eps, scale)
    return q, s, x.new_empty(x.shape, dtype=torch.float16)


# ----------------------------------------------------------------------------- norm + linear


def _rmsnorm_fp8_w4a16_linear(x, norm_weight, eps, qweight_t, scales, qzeros, bias, group_size, backend,  # type: ignore[no-untyped-def]
                              epilogue):
    """The linear (epilogue ``"none"`` or ``"silu_mul"``) on the fp16 activation of
    ``rmsnorm_fp8_quant_dequant(x, norm_weight, eps, None)`` (no counterpart in the reference):
    the GEMV stream form normalizes and quantizes x in its prologue (one launch, M <= 4); other
    configs run the norm kernel, then the linear. Bit for bit the two ops."""
    if epilogue not in ("none", "silu_mul"):
        raise ValueError(f"epilogue must be 'none' or 'silu_mul', got {epilogue!r}")
    k = x.shape[-1]
    n = qweight_t.shape[0]
    out_shape = (*x.shape[:-1], n // 2 if epilogue == "silu_mul" else n)
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    m = x2.shape[0]
    if m == 0:
        return x.new_empty(out_shape)
    _check_backend(backend)
    if _on_host("rmsnorm_fp8_w4a16_linear", x2, norm_weight, qweight_t, scales, qzeros, bias):
        _rms.check_inputs(x2, norm_weight, None)
        _, _, a = host.rmsnorm_fp8_quant_dequant(x2, norm_weight, eps, None)
        _, _, _, bias, _ = _w4a16.check_linear_args(a, qweight_t, scales, qzeros, group_size, bias, epilogue, None)
        _record_host(m, backend)
        return host.linear(a, qweight_t, scales, qzeros, bias, group_size, epilogue).reshape(out_shape)
    cfg = _decide(x2, m, n, k, group_size, backend)
    fcfg = norm_fused_config(cfg, m, n, k)
    if fcfg is not None:
        y = _w4a16.rmsnorm_fp8_w4a16_gemm_ex(
            x2, norm_weight, eps, qweight_t, scales, qzeros, group_size, fcfg, bias, epilogue
        )
    else:
        _, _, a = _rms.rmsnorm_fp8_quant_dequant(x2, norm_weight, eps, None)
        y = _w4a16.w4a16_gemm_ex(a, qweight_t, scales, qzeros, group_size, cfg, bias, epilogue)
    return y.reshape(out_shape)


@torch.library.register_fake("tokenforge::rmsnorm_fp8_w4a16_linear")
def _rmsnorm_fp8_w4a16_linear_fake(x, norm_weight, eps, qweight_t, scales, qzeros, bias, group_size, backend,  # type: ignore[no-untyped-def]
                                   epilogue):
    n = qweight_t.shape[0]
    return x.new_empty((*x.shape[:-1], n // 2 if epilogue == "silu_mul" else n))


# ----------------------------------------------------------------------------- registrations

# Each operator's Python body: the CPU kernel (the torch route) and tokenforge::_py_<op>, which
# the C++ GPU kernel calls for the calls it does not launch itself. w4a16_dequant, a load-time
# operator, has its GPU kernel here too.
_BODIES = {
    "w4a16_linear": _w4a16_linear,
    "w4a16_linear_residual": _w4a16_linear_residual,
    "w4a16_linear_silu_mul": _w4a16_linear_silu_mul,
    "w4a8_linear": _w4a8_linear,
    "rmsnorm_fp8_quant": _rmsnorm_fp8_quant,
    "rmsnorm_fp8_quant_dequant": _rmsnorm_fp8_quant_dequant,
    "rmsnorm_fp8_w4a16_linear": _rmsnorm_fp8_w4a16_linear,
}
for _name, _body in _BODIES.items():
    _schema = str(getattr(torch.ops.tokenforge, _name).default._schema)
    _LIB.define("_py_" + _schema.split("::", 1)[1])
    _LIB.impl("_py_" + _name, _body, "CompositeExplicitAutograd")
    _LIB.impl(_name, _body, "CPU")
_LIB.impl("w4a16_dequant", _w4a16_dequant, "CPU")
_LIB.impl("w4a16_dequant", _w4a16_dequant, "CUDA")
