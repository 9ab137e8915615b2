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


# Fake device addresses: 16-byte aligned, never dereferenced (every call below is rejected on
# the host before anything is launched, so this runs without a GPU).
_X, _W, _S, _Z, _O, _WS = (0x10000 * (i + 1) for i in range(6))


def test_w4a8_rejects_before_launching() -> None:
    """A W4A8 call on a GEMM config (which would first convert x into the workspace) that names
    no compiled variant is rejected with TF_EINVAL before the conversion kernel is queued; a
    launch attempt without a GPU would have returned TF_ELAUNCH instead."""
    h = _lib.lib()
    bad = _lib.TfGemmConfig(2, 96, 128, 64, 1, 4, 2)  # no such gemm_mfma tile
    rc = h.tf_w4a8_linear_ex(_X, 256, _S, 1, _W, _S, _Z, None, _O, 1152, 64, 1152, 256, 128,
                             ctypes.byref(bad), 0, None, 0, _WS, 1 << 20, None)
    assert rc == _lib.TF_EINVAL
    assert b"compiled variant" in h.tf_last_error()
    # A good config with a workspace that is too small: also rejected on the host.
    good = _lib.TfGemmConfig(2, 128, 128, 64, 2, 4, 2)
    rc = h.tf_w4a8_linear_ex(_X, 256, _S, 1, _W, _S, _Z, None, _O, 1152, 64, 1152, 256, 128,
                             ctypes.byref(good), 0, None, 0, _WS, 16, None)
    assert rc == _lib.TF_EINVAL
    assert b"workspace too small" in h.tf_last_error()
    # A GEMV config whose own launch checks fail (x of 4 rows at K = 131072 does not fit the
    # shared-x form's LDS): rejected by the variant's check, before any launch.
    gemv = _lib.TfGemmConfig(1, 16, 16, 256, 1, 4, 2)
    rc = h.tf_w4a8_linear_ex(_X, 131072, _S, 1, _W, _S, _Z, None, _O, 64, 4, 64, 131072, 128,
                             ctypes.byref(gemv), 0, None, 0, None, 0, None)
    assert rc == _lib.TF_EINVAL
    assert b"LDS" in h.tf_last_error()


def test_noalloc_rejects_a_workspace_above_its_array_on_the_host() -> None:
    h = _lib.lib()
    cfg = _lib.TfGemmConfig(2, 128, 128, 64, 8, 4, 2)
    m, n, k = 4096, 37888, 3584
    assert h.tf_w4a16_workspace_bytes_ex(m, n, k, 128, ctypes.byref(cfg), 0) > h.tf_noalloc_scratch_bytes()
    rc = h.tf_w4a16_linear_ex_noalloc(_X, k, _W, _S, _Z, None, _O, n, m, n, k, 128, ctypes.byref(cfg), 0,
                                      None, 0, None)
    assert rc == _lib.TF_EINVAL
    assert b"bytes of workspace" in h.tf_last_error()
    assert h.tf_noalloc_scratch_bytes() == 32 << 20


def test_norm_form_is_checked_before_any_launch() -> None:
    """tf_rmsnorm_fp8_quant_ex rejects an unknown form, and the row-per-wave form where it cannot
    read the rows (h % 8 != 0, h above 8192, unaligned x), on the host."""
    h = _lib.lib()
    args = (_X, 1004, _W, _O, 1004, _S, 0, None, 0, 4)  # h = 1004: not a whole number of 16-byte chunks
    assert h.tf_rmsnorm_fp8_quant_ex(*args, 1004, 1e-6, 7, None) == _lib.TF_EINVAL
    assert b"unknown form" in h.tf_last_error()
    assert h.tf_rmsnorm_fp8_quant_ex(*args, 1004, 1e-6, 2, None) == _lib.TF_EINVAL
    assert b"row-per-wave" in h.tf_last_error()
    big = (_X, 8200, _W, _O, 8200, _S, 0, None, 0, 4)
    assert h.tf_rmsnorm_fp8_quant_ex(*big, 8200, 1e-6, 2, None) == _lib.TF_EINVAL
    unaligned = (_X + 2, 1024, _W, _O, 1024, _S, 0, None, 0, 4)
    assert h.tf_rmsnorm_fp8_quant_ex(*unaligned, 1024, 1e-6, 2, None) == _lib.TF_EINVAL


def test_fp8_gemm_configs_are_w4a8_only_and_checked_before_any_launch() -> None:
    """A gemm_fp8 config is rejected by the W4A16 entry point, and by the W4A8 one where it does
    not apply (group 64, N not a multiple of 16), both on the host."""
    h = _lib.lib()
    fp8 = _lib.TfGemmConfig(3, 256, 192, 128, 1, 8, 3)
    rc = h.tf_w4a16_linear_ex(_X, 1024, _W, _S, _Z, None, _O, 1152, 256, 1152, 1024, 128, ctypes.byref(fp8), 0,
                              None, 0, None, 0, None)
    assert rc == _lib.TF_EINVAL and b"e4m3" in h.tf_last_error()
    rc = h.tf_w4a8_linear_ex(_X, 1024, _S, 1, _W, _S, _Z, None, _O, 1152, 256, 1152, 1024, 64,
                             ctypes.byref(fp8), 0, None, 0, None, 0, None)
    assert rc == _lib.TF_EINVAL and b"group_size 128" in h.tf_last_error()
    rc = h.tf_w4a8_linear_ex(_X, 1024, _S, 1, _W, _S, _Z, None, _O, 1160, 256, 1160, 1024, 128,
                             ctypes.byref(fp8), 0, None, 0, None, 0, None)
    assert rc == _lib.TF_EINVAL and b"multiple of 16" in h.tf_last_error()
