"""W4A8: the linear on FP8 activations (``tf_w4a8_linear_ex``, ``tokenforge::w4a8_linear``).

Bars:
* with a unit scale the result equals the W4A16 kernel on the decoded fp16 activations bit
  for bit (e4m3 values are exact in fp16), for the configs that decode while staging x and
  for those that decode into the workspace first — this pins the decoder on every non-NaN
  code;
* with ``rmsnorm_fp8_quant``'s per-row scales it is within the derived tolerance of the
  oracle ``w4a8_reference`` (x_scale[m] * (e4m3(x8) @ W^T) + bias, fp64), on the same
  ``x = decode * scale`` magnitudes the W4A16 bar uses;
* epilogues equal the unfused torch expressions on the W4A8 output; a NaN code gives a NaN row.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import tokenforge.kernels.ops  # noqa: F401  (registers torch.ops.tokenforge)
from oracle import pack as opack
from oracle import reference as oref
from tests.numerics import cases
from tests.numerics.tolerance import NORMWISE_MAX, contract, relative_max_error
from tokenforge.kernels.config import GemmConfig
from tokenforge.kernels.hip.rmsnorm_fp8 import rmsnorm_fp8_quant
from tokenforge.kernels.hip.w4a16 import w4a8_gemm_ex, w4a16_gemm, w4a16_gemm_ex

pytestmark = pytest.mark.gpu
G = cases.GROUP_SIZE

CONFIGS = [
    # decode while staging x
    GemmConfig("gemv_mfma", 16, 16, 128, 1, 4, 2),
    GemmConfig("gemv_mfma", 16, 16, 128, 1, 8, 2),
    GemmConfig("gemv_mfma", 16, 16, 256, 1, 4, 4),
    GemmConfig("gemv_mfma", 16, 16, 256, 1, 8, 4),
    GemmConfig("gemv_mfma", 16, 16, 128, 1, 16, 4),
    GemmConfig("gemv_mfma", 32, 32, 128, 1, 4, 2),
    GemmConfig("gemv_mfma", 16, 32, 256, 1, 4, 2),
    # decode into the workspace first
    GemmConfig("gemm_mfma", 32, 128, 128, 3, 4, 3),
    GemmConfig("gemm_mfma", 64, 128, 64, 1, 4, 2),
    GemmConfig("gemm_mfma", 256, 192, 64, 2, 8, 3),
]


def _id(c: GemmConfig) -> str:
    return f"{c.kernel}-bm{c.block_m}-bn{c.block_n}-bk{c.block_k}-sk{c.split_k}-w{c.num_warps}-st{c.num_stages}"


def _m_list(cfg: GemmConfig) -> tuple[int, ...]:
    return (1, cfg.block_m - 1, cfg.block_m + 3)


def _codes(m: int, k: int, seed: int) -> torch.Tensor:
    """Random e4m3fn codes without the two NaN codes."""
    gen = torch.Generator().manual_seed(seed)
    c = torch.randint(0, 256, (m, k), generator=gen, dtype=torch.uint8)
    c[(c & 0x7F) == 0x7F] = 0x38
    return c


@pytest.mark.parametrize("cfg", CONFIGS, ids=_id)
def test_unit_scale_equals_w4a16_on_decoded_x(cfg: GemmConfig, device: torch.device) -> None:
    n, k = 200, 512
    w = cases.on_device(cases.layer_weights(n, k, 5), device)
    b = cases.bias(n, 5).to(device)
    one = torch.ones(1, dtype=torch.float32, device=device)
    for m in _m_list(cfg):
        c = _codes(m, k, m).to(device)
        x8 = c.view(torch.float8_e4m3fn)
        y8 = w4a8_gemm_ex(x8, one, w.qweight_t, w.scales, w.qzeros, G, cfg, b)
        y16 = w4a16_gemm(x8.to(torch.float16), w.qweight_t, w.scales, w.qzeros, G, cfg, b)
        assert torch.equal(y8, y16), f"m={m}"


@pytest.mark.parametrize("cfg", CONFIGS, ids=_id)
def test_rmsnorm_fp8_output_against_oracle(cfg: GemmConfig, device: torch.device) -> None:
    n, k = 256, 512
    wn = cases.layer_weights(n, k, 6)
    w = cases.on_device(wn, device)
    b = cases.bias(n, 6)
    gamma = (torch.rand(k, generator=torch.Generator().manual_seed(1)) + 0.5).to(torch.float16)
    for m in _m_list(cfg):
        h = (torch.randn((m, k), generator=torch.Generator().manual_seed(m)) * 3).to(torch.float16)
        q8, s = rmsnorm_fp8_quant(h.to(device), gamma.to(device), 1e-6)
        y = w4a8_gemm_ex(q8, s, w.qweight_t, w.scales, w.qzeros, G, cfg, b.to(device))
        codes = q8.cpu().view(torch.uint8).numpy()
        sc = s.cpu().numpy().reshape(-1)
        ref = oref.w4a8_reference(codes, sc, wn, b.numpy())
        x_eff = oref.e4m3_decode(codes).astype(np.float64) * sc[:, None]
        y64 = y.cpu().numpy().astype(np.float64)
        tol = contract("cuda").atol(x_eff, opack.dequantize_tf(wn))
        half_ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64) / 2
        assert float((np.abs(y64 - ref) - half_ulp).max()) <= tol
        assert relative_max_error(y64, ref) <= NORMWISE_MAX


@pytest.mark.parametrize(
    "cfg",
    [GemmConfig("gemv_mfma", 16, 16, 128, 1, 16, 4), GemmConfig("gemv_mfma", 32, 32, 128, 1, 4, 2),
     GemmConfig("gemm_mfma", 256, 192, 64, 2, 8, 3)],
    ids=_id,
)
def test_epilogues_and_nan_rows(cfg: GemmConfig, device: torch.device) -> None:
    n, k, m = 400, 512, 5
    w = cases.on_device(cases.layer_weights(n, k, 9), device)
    c = _codes(m, k, 3)
    c[2, 17] = 0x7F  # a NaN code in row 2
    x8 = c.to(device).view(torch.float8_e4m3fn)
    s = torch.tensor([[0.5], [2.0], [1.0], [0.125], [3.0]], dtype=torch.float32, device=device)
    y = w4a8_gemm_ex(x8, s, w.qweight_t, w.scales, w.qzeros, G, cfg)
    assert bool(torch.isnan(y[2]).all()) and not bool(torch.isnan(y[[0, 1, 3, 4]]).any())
    fused = w4a8_gemm_ex(x8, s, w.qweight_t, w.scales, w.qzeros, G, cfg, None, "silu_mul")
    ok = [0, 1, 3, 4]
    assert torch.equal(fused[ok], (torch.nn.functional.silu(y[:, : n // 2]) * y[:, n // 2 :])[ok])
    r = cases.activations(m, n, 4).to(device)
    fr = w4a8_gemm_ex(x8, s, w.qweight_t, w.scales, w.qzeros, G, cfg, None, "residual", r)
    assert torch.equal(fr[ok], (r + y)[ok])
    # the fp16-activation path with the same epilogue and unit scale agrees too
    y16 = w4a16_gemm_ex(x8.to(torch.float16)[ok], w.qweight_t, w.scales, w.qzeros, G, cfg, None, "silu_mul")
    one = torch.ones(1, dtype=torch.float32, device=device)
    assert torch.equal(y16, w4a8_gemm_ex(x8[ok], one, w.qweight_t, w.scales, w.qzeros, G, cfg, None, "silu_mul"))


def test_op_with_leading_dims_and_static_scale(device: torch.device) -> None:
    n, k = 256, 512
    w = cases.on_device(cases.layer_weights(n, k, 11), device)
    c = _codes(6, k, 11).to(device).view(torch.float8_e4m3fn).reshape(2, 3, k)
    s = torch.tensor([0.25], dtype=torch.float32, device=device)
    y = torch.ops.tokenforge.w4a8_linear(c, s, w.qweight_t, w.scales, w.qzeros, None, G, "hip")
    assert y.shape == (2, 3, n) and y.dtype == torch.float16
    ref = torch.ops.tokenforge.w4a8_linear(c.reshape(6, k), s.reshape(1, 1).expand(6, 1).contiguous(), w.qweight_t,
                                           w.scales, w.qzeros, None, G, "hip")
    assert torch.equal(y.reshape(6, n), ref)
    with pytest.raises(TypeError, match="float8_e4m3fn"):
        w4a8_gemm_ex(c.reshape(6, k).view(torch.uint8), s, w.qweight_t, w.scales, w.qzeros, G,
                     GemmConfig("gemv_mfma", 16, 16, 128, 1, 4, 2))
    with pytest.raises(ValueError, match="one per row"):
        w4a8_gemm_ex(c.reshape(6, k), torch.ones(4, device=device), w.qweight_t, w.scales, w.qzeros, G,
                     GemmConfig("gemv_mfma", 16, 16, 128, 1, 4, 2))
