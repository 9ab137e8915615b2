"""The decode RMSNorm prologue (tf_rmsnorm_fp8_w4a16_linear) against the two ops it fuses, bit
for bit: rmsnorm_fp8_quant_dequant (dynamic scale) and then the W4A16 linear on its fp16
output, with the same config.

Every stream-form variant (waves 1..16, ring depth 2 and 4) at M = 1..4, epilogues none (with
bias) and SiLU*mul, on rows that take the kernel's fast path and rows that do not: an all-zero
row (scale 1/(448*512)), a row holding a NaN or an infinity (NaN codes, the slow encode), a row
near fp16's maximum, and rows with large outlier channels. The op routes M = 1 through the
fused kernel (ring depth 4) and larger M through the two kernels (at M = 2..4 the separate norm
kernel is faster than every workgroup normalizing the rows); both routes equal the unfused ops.
"""

from __future__ import annotations

import ctypes

import pytest
import torch
from torch.library import opcheck

import tokenforge.kernels.ops  # noqa: F401  (registers torch.ops.tokenforge)
from tests.numerics import cases
from tokenforge.kernels import _lib
from tokenforge.kernels.config import STREAM_BLOCK_K, GemmConfig
from tokenforge.kernels.hip._common import stream_of
from tokenforge.kernels.hip.rmsnorm_fp8 import rmsnorm_fp8_quant_dequant
from tokenforge.kernels.hip.w4a16 import rmsnorm_fp8_w4a16_gemm_ex, to_c_config, w4a16_gemm_ex

pytestmark = pytest.mark.gpu
G = cases.GROUP_SIZE
EPS = 1e-6

STREAM_CONFIGS = [GemmConfig("gemv_mfma", 4, 16, STREAM_BLOCK_K, 1, w, p) for p in (2, 4) for w in (1, 2, 4, 8, 16)]


def _id(c: GemmConfig) -> str:
    return f"w{c.num_warps}-p{c.num_stages}"


def _rows(m: int, k: int, seed: int, special: str, device: torch.device) -> torch.Tensor:
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn((m, k), generator=gen)
    x[:, torch.randperm(k, generator=gen)[:8]] *= 20  # outlier channels
    x = x.to(torch.float16)
    if special == "zero":
        x[0] = 0
    elif special == "nan":
        x[m - 1, k // 3] = float("nan")
    elif special == "inf":
        x[m - 1, k // 5] = float("inf")
    elif special == "large":
        x[0] = (torch.rand(k, generator=gen) * 2 - 1).to(torch.float16) * 60000
    elif special == "order":
        # A row whose fp64 sum of squares depends on the order of the adds: 1024^2, 0.25^2 and
        # two tiny squares (154 * 2^-24)^2 half a row away; two forms adding in different orders
        # round var differently.
        x[0] = 0
        x[0, 0], x[0, 2] = 1024, 0.25
        x[0, k // 2] = x[0, k // 2 + 2] = 154 * 2.0**-24
    return x.to(device)


def _gamma(k: int, seed: int, device: torch.device) -> torch.Tensor:
    gen = torch.Generator().manual_seed(1000 + seed)
    return (1 + 0.1 * torch.randn(k, generator=gen)).to(torch.float16).to(device)


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int16)


@pytest.mark.parametrize("cfg", STREAM_CONFIGS, ids=_id)
def test_fused_equals_norm_then_linear(cfg: GemmConfig, device: torch.device) -> None:
    n, k = 512, 2048  # K / 128 = 16 steps: every wave count takes part
    w = cases.on_device(cases.layer_weights(n, k, 4), device)
    b = cases.bias(n, 4).to(device)
    gamma = _gamma(k, 0, device)
    for m in (1, 2, 3, 4):
        for special in ("none", "zero", "nan", "inf", "large", "order"):
            x = _rows(m, k, 10 * m + len(special), special, device)
            _, _, a = rmsnorm_fp8_quant_dequant(x, gamma, EPS)
            for epilogue, bias in (("none", b), ("silu_mul", None)):
                ref = w4a16_gemm_ex(a, w.qweight_t, w.scales, w.qzeros, G, cfg, bias, epilogue)
                got = rmsnorm_fp8_w4a16_gemm_ex(x, gamma, EPS, w.qweight_t, w.scales, w.qzeros, G, cfg, bias, epilogue)
                assert got.shape == ref.shape
                assert torch.equal(_bits(got), _bits(ref)), f"m={m} rows={special} epilogue={epilogue}"


def test_fused_at_the_decode_shapes(device: torch.device) -> None:
    """qkv (4608 x 3584, bias) and gate_up (37888 x 3584, SiLU*mul) at M = 1 and 4 through the op,
    against the two unfused ops (the shapes the decode stack runs)."""
    ops = torch.ops.tokenforge
    gamma = _gamma(3584, 1, device)
    for n, epilogue, seed in ((4608, "none", 5), (37888, "silu_mul", 6)):
        w = cases.on_device(cases.layer_weights(n, 3584, seed), device)
        b = cases.bias(n, seed).to(device) if epilogue == "none" else None
        for m in (1, 4):
            x = _rows(m, 3584, seed + m, "none", device)
            _, _, a = ops.rmsnorm_fp8_quant_dequant(x, gamma, EPS, None)
            if epilogue == "none":
                ref = ops.w4a16_linear(a, w.qweight_t, w.scales, w.qzeros, b, G, "hip")
            else:
                ref = ops.w4a16_linear_silu_mul(a, w.qweight_t, w.scales, w.qzeros, b, G, "hip")
            got = ops.rmsnorm_fp8_w4a16_linear(x, gamma, EPS, w.qweight_t, w.scales, w.qzeros, b, G, "hip", epilogue)
            assert torch.equal(got, ref), f"n={n} m={m}"


def test_op_routes_larger_m_through_two_kernels(device: torch.device) -> None:
    n, k = 1024, 1024
    w = cases.on_device(cases.layer_weights(n, k, 7), device)
    gamma = _gamma(k, 2, device)
    ops = torch.ops.tokenforge
    for m in (1, 5, 40):
        x = _rows(m, k, 70 + m, "none", device).reshape(1, m, k)
        _, _, a = ops.rmsnorm_fp8_quant_dequant(x, gamma, EPS, None)
        ref = ops.w4a16_linear_silu_mul(a, w.qweight_t, w.scales, w.qzeros, None, G, "hip")
        got = ops.rmsnorm_fp8_w4a16_linear(x, gamma, EPS, w.qweight_t, w.scales, w.qzeros, None, G, "hip", "silu_mul")
        assert got.shape == (1, m, n // 2)
        assert torch.equal(got, ref), f"m={m}"


def test_op_falls_back_where_the_prologue_does_not_fit(device: torch.device) -> None:
    """M = 4, K = 12160: the stream form stages this x, but the prologue's scratch does not fit
    beside it (and K is past the prologue's 8192): the op runs the two kernels, same bits."""
    from tokenforge.kernels.config import stream_form_applies

    n, k = 256, 12160
    assert stream_form_applies(4, n, k, 8) and not stream_form_applies(4, n, k, 8, norm=True)
    w = cases.on_device(cases.layer_weights(n, k, 11), device)
    gamma = _gamma(k, 3, device)
    ops = torch.ops.tokenforge
    x = _rows(4, k, 77, "order", device)
    _, _, a = ops.rmsnorm_fp8_quant_dequant(x, gamma, EPS, None)
    ref = ops.w4a16_linear(a, w.qweight_t, w.scales, w.qzeros, None, G, "hip")
    got = ops.rmsnorm_fp8_w4a16_linear(x, gamma, EPS, w.qweight_t, w.scales, w.qzeros, None, G, "hip", "none")
    assert torch.equal(got, ref)


def test_opcheck(device: torch.device) -> None:
    w = cases.on_device(cases.layer_weights(64, 256, 0), device)
    x = cases.activations(3, 256, 0).to(device)
    gamma = torch.ones(256, dtype=torch.float16, device=device)
    b = cases.bias(64, 0).to(device)
    opcheck(
        torch.ops.tokenforge.rmsnorm_fp8_w4a16_linear.default,
        (x, gamma, EPS, w.qweight_t, w.scales, w.qzeros, b, G, "hip", "none"),
        test_utils=("test_schema", "test_faketensor", "test_aot_dispatch_dynamic"),
    )


def test_rejections(device: torch.device) -> None:
    n, k = 256, 512
    w = cases.on_device(cases.layer_weights(n, k, 8), device)
    x = cases.activations(2, k, 8).to(device)
    gamma = torch.ones(k, dtype=torch.float16, device=device)
    kgemv = GemmConfig("gemv_mfma", 16, 16, 128, 1, 4, 2)
    with pytest.raises(ValueError, match="stream form"):
        rmsnorm_fp8_w4a16_gemm_ex(x, gamma, EPS, w.qweight_t, w.scales, w.qzeros, G, kgemv)
    stream = STREAM_CONFIGS[2]
    with pytest.raises(ValueError, match="epilogue"):
        rmsnorm_fp8_w4a16_gemm_ex(x, gamma, EPS, w.qweight_t, w.scales, w.qzeros, G, stream, None, "residual")
    with pytest.raises(ValueError, match="norm weight shape"):
        rmsnorm_fp8_w4a16_gemm_ex(x, gamma[:-8], EPS, w.qweight_t, w.scales, w.qzeros, G, stream)
    with pytest.raises(ValueError, match="epilogue"):
        torch.ops.tokenforge.rmsnorm_fp8_w4a16_linear(x, gamma, EPS, w.qweight_t, w.scales, w.qzeros, None, G, "hip",
                                                       "residual")
    # The C ABI rejects a config that is not the stream form, an M above 4 and a null norm
    # weight before launching anything.
    out = torch.empty((5, n), dtype=torch.float16, device=device)
    x5 = cases.activations(5, k, 9).to(device)
    h = _lib.lib()
    for cfg, m, gptr in ((kgemv, 2, gamma.data_ptr()), (stream, 5, gamma.data_ptr()), (stream, 2, None)):
        c = to_c_config(cfg)
        rc = h.tf_rmsnorm_fp8_w4a16_linear(
            x5.data_ptr(), k, gptr, EPS, w.qweight_t.data_ptr(), w.scales.data_ptr(), w.qzeros.data_ptr(), None,
            out.data_ptr(), n, m, n, k, G, ctypes.byref(c), _lib.EPILOGUE_NONE, stream_of(device),
        )
        assert rc == 1, (cfg, m)
    torch.cuda.synchronize()
