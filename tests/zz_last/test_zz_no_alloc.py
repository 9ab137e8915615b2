"""tf_w4a16_linear_ex_noalloc: the linear with its workspace in the library's fixed device array.

Called through the C ABI and compared bit for bit with tf_w4a16_linear_ex (same kernels, a
torch-allocated workspace) on two calls in a row, the second with a smaller M, for configs
whose kernels use the workspace: split-K partials of the two-buffer and pipelined GEMMs, and
the fp32 rows through which the LDS-tile GEMMs reduce a SiLU*mul epilogue.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from tests.numerics import cases
from tokenforge.kernels import _lib
from tokenforge.kernels.config import GemmConfig
from tokenforge.kernels.hip.w4a16 import EPILOGUES, to_c_config, w4a16_gemm_ex

pytestmark = pytest.mark.gpu
G = cases.GROUP_SIZE

CONFIGS = [
    (GemmConfig("gemm_mfma", 128, 128, 64, 4, 4, 2), "none"),
    (GemmConfig("gemm_mfma", 256, 128, 64, 2, 8, 3), "none"),
    (GemmConfig("gemm_mfma", 64, 128, 128, 3, 4, 3), "residual"),
    (GemmConfig("gemm_mfma", 128, 128, 64, 1, 4, 2), "silu_mul"),
]


def _noalloc(x, w, cfg, epilogue, residual=None):  # type: ignore[no-untyped-def]
    m, k = x.shape
    n = w.qweight_t.shape[0]
    n_out = n // 2 if epilogue == "silu_mul" else n
    out = torch.empty((m, n_out), dtype=torch.float16, device=x.device)
    c = to_c_config(cfg)
    rc = _lib.lib().tf_w4a16_linear_ex_noalloc(
        x.data_ptr(), k, w.qweight_t.data_ptr(), w.scales.data_ptr(), w.qzeros.data_ptr(), None,
        out.data_ptr(), n_out, m, n, k, G, ctypes.byref(c), EPILOGUES[epilogue],
        None if residual is None else residual.data_ptr(), n, torch.cuda.current_stream().cuda_stream,
    )
    _lib.check(rc, "tf_w4a16_linear_ex_noalloc")
    return out


@pytest.mark.parametrize(("cfg", "epilogue"), CONFIGS, ids=lambda v: str(v))
def test_noalloc_equals_the_workspace_entry_point(cfg: GemmConfig, epilogue: str, device: torch.device) -> None:
    n, k = 1152, 896
    w = cases.on_device(cases.layer_weights(n, k, 0), device)
    h = _lib.lib()
    for m in (200, 37):  # the second call is smaller; the array keeps the first call's contents
        x = cases.activations(m, k, m).to(device)
        r = (torch.randn((m, n), device=device) * 0.1).to(torch.float16) if epilogue == "residual" else None
        need = h.tf_w4a16_workspace_bytes_ex(m, n, k, G, ctypes.byref(to_c_config(cfg)), EPILOGUES[epilogue])
        assert 0 < need <= h.tf_noalloc_scratch_bytes(), (cfg, m, need)
        want = w4a16_gemm_ex(x, w.qweight_t, w.scales, w.qzeros, G, cfg, None, epilogue,
                             None if r is None else r.clone())
        got = _noalloc(x, w, cfg, epilogue, None if r is None else r.clone())
        torch.cuda.synchronize()
        assert torch.equal(got, want), (cfg, epilogue, m)


def test_noalloc_rejects_a_workspace_above_its_array(device: torch.device) -> None:
    n, k = 1152, 896
    w = cases.on_device(cases.layer_weights(n, k, 0), device)
    cfg = GemmConfig("gemm_mfma", 128, 128, 64, 7, 4, 2)
    m = 4096  # 7 * 4096 * 1152 * 4 bytes of partials: above 32 MiB
    x = cases.activations(m, k, 1).to(device)
    with pytest.raises(ValueError, match="bytes of workspace"):
        _noalloc(x, w, cfg, "none")
