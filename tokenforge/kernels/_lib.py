"""ctypes binding of ``libtokenforge_hip.so``, the C ABI declared in ``include/tokenforge_hip.h``.

This module only loads the library and converts its status codes into exceptions; it never
computes anything itself. Loading works without a GPU (the library only links the HIP
runtime), so the CPU test tier can check that every declared symbol is exported.
"""

from __future__ import annotations

import ctypes
import functools
import os
from pathlib import Path

ABI_VERSION = 7
"""Must equal ``tf_abi_version()`` of the loaded library."""

LIB_ENV = "TOKENFORGE_HIP_LIB"
LIB_PATH = Path(__file__).resolve().parents[2] / "tokenforge_amd" / "lib" / "libtokenforge_hip.so"

TF_OK = 0
TF_EINVAL = 1
TF_ELAUNCH = 2
TF_ERANGE = 3

KERNEL_IDS = {"gemv_dot": 0, "gemv_mfma": 1, "gemm_mfma": 2, "gemm_fp8": 3}
EPILOGUE_NONE = 0
EPILOGUE_RESIDUAL = 1
EPILOGUE_SILU_MUL = 2
KERNEL_NAMES = {v: k for k, v in KERNEL_IDS.items()}


class TfGemmConfig(ctypes.Structure):
    """``tf_gemm_config`` (all int32)."""

    _fields_ = [
        ("kernel", ctypes.c_int32),
        ("block_m", ctypes.c_int32),
        ("block_n", ctypes.c_int32),
        ("block_k", ctypes.c_int32),
        ("split_k", ctypes.c_int32),
        ("num_warps", ctypes.c_int32),
        ("num_stages", ctypes.c_int32),
    ]


class HipLibraryError(RuntimeError):
    """The HIP kernel library is missing, stale, or failed to load."""


class HipLaunchError(RuntimeError):
    """HIP reported an error when a kernel was launched."""


_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

# name -> (restype, argtypes), in the order of include/tokenforge_hip.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "tf_abi_version": (ctypes.c_int, []),
    "tf_last_error": (ctypes.c_char_p, []),
    "tf_pack_int4": (ctypes.c_int, [_p, _p, _i64, _i64, _p, _p]),
    "tf_unpack_int4": (ctypes.c_int, [_p, _p, _i64, _i64, _p]),
    "tf_awq_to_tf": (ctypes.c_int, [_p, _p, _i64, _i64, _p]),
    "tf_tf_to_awq": (ctypes.c_int, [_p, _p, _i64, _i64, _p]),
    "tf_tile_pack": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _p]),
    "tf_tile_unpack": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _p]),
    "tf_awq_quantize": (ctypes.c_int, [_p, _i64, _i64, _i32, _p, _p, _p, _p]),
    "tf_w4a16_dequant": (ctypes.c_int, [_p, _p, _p, _p, _i64, _i64, _i32, _p]),
    "tf_num_variants": (ctypes.c_int, []),
    "tf_get_variant": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(TfGemmConfig)]),
    "tf_w4a16_workspace_bytes": (_i64, [_i64, _i64, _i64, _i32, ctypes.POINTER(TfGemmConfig)]),
    "tf_w4a16_linear": (
        ctypes.c_int,
        [_p, _i64, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32,
         ctypes.POINTER(TfGemmConfig), _p, _i64, _p],
    ),
    "tf_w4a16_workspace_bytes_ex": (_i64, [_i64, _i64, _i64, _i32, ctypes.POINTER(TfGemmConfig), _i32]),
    "tf_w4a16_linear_ex": (
        ctypes.c_int,
        [_p, _i64, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32,
         ctypes.POINTER(TfGemmConfig), _i32, _p, _i64, _p, _i64, _p],
    ),
    "tf_noalloc_scratch_bytes": (_i64, []),
    "tf_w4a16_linear_ex_noalloc": (
        ctypes.c_int,
        [_p, _i64, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32,
         ctypes.POINTER(TfGemmConfig), _i32, _p, _i64, _p],
    ),
    "tf_w4a8_workspace_bytes_ex": (_i64, [_i64, _i64, _i64, _i32, ctypes.POINTER(TfGemmConfig), _i32]),
    "tf_w4a8_linear_ex": (
        ctypes.c_int,
        [_p, _i64, _p, _i64, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32,
         ctypes.POINTER(TfGemmConfig), _i32, _p, _i64, _p, _i64, _p],
    ),
    "tf_rmsnorm_fp8_quant": (ctypes.c_int, [_p, _i64, _p, _p, _i64, _p, _i32, _i64, _i64, _f32, _p]),
    "tf_rmsnorm_fp8_quant_dq": (ctypes.c_int, [_p, _i64, _p, _p, _i64, _p, _i32, _p, _i64, _i64, _i64, _f32, _p]),
    "tf_rmsnorm_fp8_quant_ex": (
        ctypes.c_int, [_p, _i64, _p, _p, _i64, _p, _i32, _p, _i64, _i64, _i64, _f32, _i32, _p]),
    "tf_rmsnorm_fp8_w4a16_linear": (
        ctypes.c_int,
        [_p, _i64, _p, _f32, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32,
         ctypes.POINTER(TfGemmConfig), _i32, _p]),
    "tf_e4m3_encode": (ctypes.c_int, [_p, _p, _i64, _p]),
}


def library_path() -> Path:
    env = os.environ.get(LIB_ENV)
    return Path(env) if env else LIB_PATH


TORCH_OPS_PATH = LIB_PATH.parent / "libtokenforge_torch.so"


def torch_ops_path() -> Path:
    """The torch operator extension (``tokenforge_amd/ext/torch_ops.cpp``), beside the library."""
    return TORCH_OPS_PATH


@functools.cache
def lib() -> ctypes.CDLL:
    """Load the library once per process. Raises :class:`HipLibraryError` when missing."""
    path = library_path()
    if not path.exists():
        raise HipLibraryError(
            f"{path} is missing: build it with `python -m tokenforge_amd.build` "
            "(tokenforge.kernels has no CPU or fallback path)"
        )
    try:
        handle = ctypes.CDLL(str(path))
    except OSError as exc:
        raise HipLibraryError(f"cannot load {path}: {exc}") from exc
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    got = handle.tf_abi_version()
    if got != ABI_VERSION:
        raise HipLibraryError(f"{path} has ABI {got}, this package expects {ABI_VERSION}: rebuild it")
    return handle


def available() -> bool:
    try:
        lib()
    except HipLibraryError:
        return False
    return True


def check(rc: int, what: str) -> None:
    """Raise the exception matching a ``tf_*`` status code."""
    if rc == TF_OK:
        return
    msg = lib().tf_last_error().decode(errors="replace") or what
    if rc in (TF_EINVAL, TF_ERANGE):
        raise ValueError(msg)
    raise HipLaunchError(msg)


def variants() -> list[TfGemmConfig]:
    """Every compiled (kernel, block_m, block_n, block_k, num_warps, num_stages) variant."""
    h = lib()
    out = []
    for i in range(h.tf_num_variants()):
        cfg = TfGemmConfig()
        check(h.tf_get_variant(i, ctypes.byref(cfg)), "tf_get_variant")
        out.append(cfg)
    return out
