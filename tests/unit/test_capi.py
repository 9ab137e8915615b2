"""T0: the C-ABI library loads and exports every entry point ``include/*.h`` declares.

Runs on CPU: loading the library needs only the HIP runtime, and no test here launches a
kernel. The Python-side variant table must equal the table compiled into the library.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

from tokenforge.kernels import _lib
from tokenforge.kernels.config import VARIANTS

INCLUDE = Path(__file__).resolve().parents[2] / "include"


def _declared_functions() -> set[str]:
    names: set[str] = set()
    for header in INCLUDE.glob("*.h"):
        text = header.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(tf_[a-z0-9_]+)\s*\(", text))
    return names


def test_header_declares_the_bound_signatures() -> None:
    declared = _declared_functions()
    assert declared, "no tf_* declarations found"
    assert declared == set(_lib.SIGNATURES), "ctypes signatures and the header disagree"


def test_library_exports_every_declared_symbol() -> None:
    handle = ctypes.CDLL(str(_lib.library_path()))
    missing = [name for name in _declared_functions() if not hasattr(handle, name)]
    assert not missing, f"not exported: {missing}"


def test_abi_version_and_error_string() -> None:
    h = _lib.lib()
    assert h.tf_abi_version() == _lib.ABI_VERSION
    assert isinstance(h.tf_last_error(), bytes)


def test_variant_table_matches_python() -> None:
    compiled = [
        (_lib.KERNEL_NAMES[v.kernel], v.block_m, v.block_n, v.block_k, v.num_warps, v.num_stages)
        for v in _lib.variants()
    ]
    assert compiled == list(VARIANTS)
    assert all(v.split_k == 1 for v in _lib.variants())


def test_variant_lookup_rejects_bad_index() -> None:
    h = _lib.lib()
    cfg = _lib.TfGemmConfig()
    assert h.tf_get_variant(-1, ctypes.byref(cfg)) == _lib.TF_EINVAL
    assert b"out of range" in h.tf_last_error()


def test_workspace_query_is_host_only() -> None:
    """Workspace sizing is pure host arithmetic: split-K GEMM needs S*M*N fp32."""
    h = _lib.lib()
    gemm = _lib.TfGemmConfig(2, 128, 128, 64, 4, 4, 2)
    assert h.tf_w4a16_workspace_bytes(256, 3584, 18944, 128, ctypes.byref(gemm)) == 4 * 256 * 3584 * 4
    gemv = _lib.TfGemmConfig(1, 16, 16, 128, 1, 8, 2)
    assert h.tf_w4a16_workspace_bytes(1, 3584, 3584, 128, ctypes.byref(gemv)) == 0
    unknown = _lib.TfGemmConfig(2, 96, 128, 64, 1, 4, 2)
    assert h.tf_w4a16_workspace_bytes(256, 3584, 3584, 128, ctypes.byref(unknown)) == 0
