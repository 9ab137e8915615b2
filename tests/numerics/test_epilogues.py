"""Fused epilogues of the W4A16 linear against their unfused torch expressions, bit for bit.

* residual: ``residual + y`` (torch fp16 add of the fp16 linear output);
* silu_mul: ``silu(y[:, :N/2]) * y[:, N/2:]`` (torch fp16 silu and multiply).

Every kernel family and its variants take part: the GEMV kernels and the register-streamed
GEMM pair gate and up columns inside a tile (lanes c and c ^ 8), the LDS-tile GEMMs and every
split-K launch reduce through fp32 partials. Same config for the fused and the unfused run,
so ``y`` is the same bits in both.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

import tokenforge.kernels.ops  # noqa: F401  (registers torch.ops.tokenforge)
from tests.numerics import cases
from tokenforge.kernels import _lib
from tokenforge.kernels.config import GemmConfig
from tokenforge.kernels.hip._common import stream_of
from tokenforge.kernels.hip.w4a16 import to_c_config, w4a16_gemm, w4a16_gemm_ex

pytestmark = pytest.mark.gpu
G = cases.GROUP_SIZE

CONFIGS = [
    GemmConfig("gemv_mfma", 16, 16, 128, 1, 4, 2),
    GemmConfig("gemv_mfma", 16, 32, 128, 1, 2, 2),
    GemmConfig("gemv_mfma", 16, 16, 128, 1, 8, 2),
    GemmConfig("gemv_mfma", 16, 16, 256, 1, 4, 4),
    GemmConfig("gemv_mfma", 16, 16, 256, 1, 8, 4),
    GemmConfig("gemv_mfma", 16, 16, 256, 1, 4, 2),
    GemmConfig("gemv_mfma", 16, 16, 128, 1, 16, 4),
    GemmConfig("gemv_mfma", 16, 64, 128, 1, 2, 2),
    GemmConfig("gemv_mfma", 16, 32, 256, 1, 4, 2),
    GemmConfig("gemv_mfma", 16, 64, 128, 1, 4, 2),
    GemmConfig("gemv_mfma", 32, 32, 128, 1, 4, 2),
    GemmConfig("gemm_mfma", 64, 128, 64, 1, 4, 2),
    GemmConfig("gemm_mfma", 128, 128, 32, 2, 4, 2),
    GemmConfig("gemm_mfma", 256, 192, 64, 1, 8, 3),
    GemmConfig("gemm_mfma", 128, 256, 64, 3, 8, 3),
    GemmConfig("gemm_mfma", 16, 64, 128, 1, 4, 3),
    GemmConfig("gemm_mfma", 32, 128, 128, 3, 4, 3),
    GemmConfig("gemm_mfma", 64, 256, 128, 1, 4, 3),
    GemmConfig("gemm_mfma", 256, 160, 128, 2, 4, 2),
]


def _id(c: GemmConfig) -> str:
    return f"{c.kernel}-bm{c.block_m}-bn{c.block_n}-bk{c.block_k}-sk{c.split_k}-w{c.num_warps}-st{c.num_stages}"


def _m_list(cfg: GemmConfig) -> tuple[int, ...]:
    return (1, cfg.block_m - 1, cfg.block_m + 3)


@pytest.mark.parametrize("cfg", CONFIGS, ids=_id)
def test_silu_mul_and_residual_equal_unfused(cfg: GemmConfig, device: torch.device) -> None:
    n, k = 400, 512  # N/2 = 200: ragged against every tile width
    w = cases.on_device(cases.layer_weights(n, k, 0), device)
    b = cases.bias(n, 0).to(device)
    inter = n // 2
    for m in _m_list(cfg):
        x = cases.activations(m, k, 0).to(device)
        y = w4a16_gemm(x, w.qweight_t, w.scales, w.qzeros, G, cfg, b)
        fused = w4a16_gemm_ex(x, w.qweight_t, w.scales, w.qzeros, G, cfg, b, "silu_mul")
        assert fused.shape == (m, inter)
        assert torch.equal(fused, torch.nn.functional.silu(y[:, :inter]) * y[:, inter:]), f"silu_mul m={m}"
        r = cases.activations(m, n, 1).to(device)
        fused_r = w4a16_gemm_ex(x, w.qweight_t, w.scales, w.qzeros, G, cfg, b, "residual", r)
        assert torch.equal(fused_r, r + y), f"residual m={m}"


def test_residual_in_place_through_the_c_abi(device: torch.device) -> None:
    """out may be the residual itself (x += linear(...))."""
    n, k, m = 256, 512, 5
    w = cases.on_device(cases.layer_weights(n, k, 2), device)
    x = cases.activations(m, k, 2).to(device)
    cfg = GemmConfig("gemv_mfma", 16, 32, 128, 1, 4, 2)
    h = torch.randn((m, n), device=device).to(torch.float16)
    expect = h + w4a16_gemm(x, w.qweight_t, w.scales, w.qzeros, G, cfg)
    c = to_c_config(cfg)
    rc = _lib.lib().tf_w4a16_linear_ex(
        x.data_ptr(), k, w.qweight_t.data_ptr(), w.scales.data_ptr(), w.qzeros.data_ptr(), None,
        h.data_ptr(), n, m, n, k, G, ctypes.byref(c), _lib.EPILOGUE_RESIDUAL, h.data_ptr(), n, None, 0,
        stream_of(device),
    )
    _lib.check(rc, "tf_w4a16_linear_ex")
    torch.cuda.synchronize()
    assert torch.equal(h, expect)


def test_ops_match_unfused_ops(device: torch.device) -> None:
    n, k = 1024, 512
    w = cases.on_device(cases.layer_weights(n, k, 3), device)
    ops = torch.ops.tokenforge
    for m in (1, 7, 40, 300):
        x = cases.activations(m, k, 3).to(device).reshape(1, m, k)
        y = ops.w4a16_linear(x, w.qweight_t, w.scales, w.qzeros, None, G, "hip")
        s = ops.w4a16_linear_silu_mul(x, w.qweight_t, w.scales, w.qzeros, None, G, "hip")
        assert s.shape == (1, m, n // 2)
        assert torch.equal(s, torch.nn.functional.silu(y[..., : n // 2]) * y[..., n // 2 :])
        r = torch.randn((1, m, n), device=device).to(torch.float16)
        assert torch.equal(ops.w4a16_linear_residual(x, w.qweight_t, w.scales, w.qzeros, None, r, G, "hip"), r + y)


def test_epilogue_argument_errors(device: torch.device) -> None:
    w = cases.on_device(cases.layer_weights(200, 256, 0), device)
    x = cases.activations(3, 256, 0).to(device)
    cfg = GemmConfig("gemv_mfma", 16, 16, 128, 1, 1, 2)
    with pytest.raises(ValueError, match="multiple of 16"):
        w4a16_gemm_ex(x, w.qweight_t, w.scales, w.qzeros, G, cfg, None, "silu_mul")
    with pytest.raises(ValueError, match="residual of shape"):
        w4a16_gemm_ex(x, w.qweight_t, w.scales, w.qzeros, G, cfg, None, "residual")
    with pytest.raises(ValueError, match="epilogue must be one of"):
        w4a16_gemm_ex(x, w.qweight_t, w.scales, w.qzeros, G, cfg, None, "gelu")
    c = to_c_config(cfg)
    out = torch.empty((3, 200), dtype=torch.float16, device=device)
    rc = _lib.lib().tf_w4a16_linear_ex(
        x.data_ptr(), 256, w.qweight_t.data_ptr(), w.scales.data_ptr(), w.qzeros.data_ptr(), None,
        out.data_ptr(), 200, 3, 200, 256, G, ctypes.byref(c), 7, None, 0, None, 0, stream_of(device),
    )
    assert rc == _lib.TF_EINVAL and b"unknown epilogue" in _lib.lib().tf_last_error()
    rc = _lib.lib().tf_w4a16_linear_ex(
        x.data_ptr(), 256, w.qweight_t.data_ptr(), w.scales.data_ptr(), w.qzeros.data_ptr(), None,
        out.data_ptr(), 200, 3, 200, 256, G, ctypes.byref(c), _lib.EPILOGUE_RESIDUAL, None, 200, None, 0,
        stream_of(device),
    )
    assert rc == _lib.TF_EINVAL and b"needs a residual" in _lib.lib().tf_last_error()
