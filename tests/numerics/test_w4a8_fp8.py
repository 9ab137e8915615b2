"""The W4A8 fp8 GEMM (``gemm_fp8``: e4m3 x on the fp8 MFMA, exact e4m3 (q - z), the group scale
applied in fp32 after each 128-K group) against the oracle.

Bars: within the derived bound ``c sqrt(K) eps16 max|x| max|w|`` plus half an fp16 ulp of the
output (the result is rounded to fp16 once) of ``oracle.reference.w4a8_exact_reference`` (fp64,
weights never rounded), and within 1e-2 normwise of both that and ``w4a8_reference`` (the
fp16-weight form the other W4A8 kernels compute); the residual and SiLU*mul epilogues equal
the torch composition of the kernel's own plain output bit for bit; reruns are bit-identical;
the ops path picks the fp8 GEMM at prefill M. Inputs: the numerics suite's seeded weights and
the FP8 codes ``rmsnorm_fp8_reference`` makes of seeded activations (per-row scales).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import tokenforge.kernels.ops  # noqa: F401  (registers torch.ops.tokenforge)
from oracle import pack as opack
from oracle import reference as oref
from tests.numerics import cases
from tests.numerics.tolerance import EPS_FP16, NORMWISE_MAX, contract, relative_max_error
from tokenforge.kernels.config import FP8_PC_TILES, FP8_TILES, GemmConfig, fp8_gemm_applies, fp8_gemm_config
from tokenforge.kernels.hip.w4a16 import w4a8_gemm_ex

pytestmark = pytest.mark.gpu
G = 128
FP8_CONFIGS = ([GemmConfig("gemm_fp8", bm, bn, 128, 1, wm * wn, s + 1) for bm, bn, wm, wn, s in FP8_TILES]
               + [GemmConfig("gemm_fp8", bm, bn, 128, 1, wm * wn, 8) for bm, bn, wm, wn in FP8_PC_TILES])


def _codes(m: int, k: int, seed: int) -> tuple[np.ndarray, np.ndarray]:
    """FP8 codes and per-row scales as rmsnorm_fp8_quant makes them (outlier channels x20)."""
    x = cases.activations(m, k, seed).numpy().astype(np.float32)
    x[:, :: max(1, k // 8)] *= 20
    gamma = np.ones(k, dtype=np.float16)
    q, s = oref.rmsnorm_fp8_reference(x.astype(np.float16), gamma, 1e-6)
    return q, s.reshape(-1)


def _check(y: torch.Tensor, codes: np.ndarray, xs: np.ndarray, w: opack.W4A16Weights, what: str,
           bias: np.ndarray | None = None) -> None:
    yn = y.float().cpu().numpy().astype(np.float64)
    exact = oref.w4a8_exact_reference(codes, xs, w, bias)
    x_eff = oref.e4m3_decode(codes).astype(np.float64) * xs.reshape(-1, 1).astype(np.float64)
    wmax = float(np.abs(opack.dequantize_tf(w).astype(np.float64)).max())
    tol = contract("cuda").c * math.sqrt(codes.shape[1]) * EPS_FP16 * float(np.abs(x_eff).max()) * wmax
    half_ulp = np.spacing(np.abs(exact).astype(np.float16)).astype(np.float64) / 2
    excess = float((np.abs(yn - exact) - half_ulp).max())
    assert excess <= tol, f"{what}: error {excess:.3e} above half an ulp exceeds the derived bound {tol:.3e}"
    assert relative_max_error(yn, exact) <= NORMWISE_MAX, what
    assert relative_max_error(yn, oref.w4a8_reference(codes, xs, w, bias)) <= NORMWISE_MAX, what


def _run(codes: np.ndarray, xs: np.ndarray, w: opack.W4A16Weights, cfg: GemmConfig, device: torch.device,
         bias: torch.Tensor | None = None, epilogue: str = "none", residual: torch.Tensor | None = None) -> torch.Tensor:
    wd = cases.on_device(w, device)
    x8 = torch.from_numpy(codes).to(device).view(torch.float8_e4m3fn)
    s = torch.from_numpy(xs.astype(np.float32)).to(device)
    return w4a8_gemm_ex(x8, s, wd.qweight_t, wd.scales, wd.qzeros, G, cfg, bias, epilogue, residual)


@pytest.mark.parametrize("cfg", FP8_CONFIGS, ids=str)
@pytest.mark.parametrize(("m", "n", "k"), [(256, 1152, 896), (300, 9728, 896), (64, 896, 4864), (513, 384, 1024)])
def test_against_the_exact_oracle(cfg: GemmConfig, m: int, n: int, k: int, device: torch.device) -> None:
    w = cases.layer_weights(n, k, 0)
    codes, xs = _codes(m, k, seed=m)
    for split in (1, 4):
        c = GemmConfig(cfg.kernel, cfg.block_m, cfg.block_n, cfg.block_k, split, cfg.num_warps, cfg.num_stages)
        y = _run(codes, xs, w, c, device)
        assert y.shape == (m, n)
        _check(y, codes, xs, w, f"{c} M={m} N={n} K={k}")
        assert torch.equal(y, _run(codes, xs, w, c, device)), f"{c}: reruns differ"


@pytest.mark.parametrize("cfg", [FP8_CONFIGS[0], FP8_CONFIGS[3]], ids=str)
def test_bias_and_epilogues(cfg: GemmConfig, device: torch.device) -> None:
    m, n, k = 256, 2304, 1024
    w = cases.layer_weights(n, k, 3)
    codes, xs = _codes(m, k, seed=3)
    bias = cases.bias(n, 3)
    y = _run(codes, xs, w, cfg, device, bias=bias.to(device))
    _check(y, codes, xs, w, f"{cfg} bias", bias.numpy())
    gen = torch.Generator().manual_seed(4)
    res = (torch.randn((m, n), generator=gen) * 0.5).to(torch.float16).to(device)
    yr = _run(codes, xs, w, cfg, device, bias=bias.to(device), epilogue="residual", residual=res)
    assert torch.equal(yr, res + y)
    ys = _run(codes, xs, w, cfg, device, bias=bias.to(device), epilogue="silu_mul")
    assert torch.equal(ys, torch.nn.functional.silu(y[:, : n // 2]) * y[:, n // 2:])
    split = GemmConfig(cfg.kernel, cfg.block_m, cfg.block_n, cfg.block_k, 2, cfg.num_warps, cfg.num_stages)
    ys2 = _run(codes, xs, w, split, device, bias=bias.to(device), epilogue="silu_mul")
    y2 = _run(codes, xs, w, split, device, bias=bias.to(device))
    assert torch.equal(ys2, torch.nn.functional.silu(y2[:, : n // 2]) * y2[:, n // 2:])


def test_static_scale_and_nan_rows(device: torch.device) -> None:
    m, n, k = 128, 512, 512
    w = cases.layer_weights(n, k, 5)
    codes, _ = _codes(m, k, seed=5)
    xs = np.array([0.02], dtype=np.float32)
    cfg = FP8_CONFIGS[4]
    y = _run(codes, xs, w, cfg, device)
    _check(y, codes, xs, w, "static scale")
    codes_nan = codes.copy()
    codes_nan[7, 100] = 0x7F  # NaN code: its row turns NaN, the others are untouched
    yn = _run(codes_nan, xs, w, cfg, device)
    assert bool(torch.isnan(yn[7]).all())
    keep = torch.ones(m, dtype=torch.bool)
    keep[7] = False
    assert torch.equal(yn[keep], y[keep])


def test_the_op_runs_the_fp8_gemm_at_prefill_m(device: torch.device) -> None:
    m, n, k = 256, 4608, 3584
    assert fp8_gemm_applies(256, n, k, G)
    assert not fp8_gemm_applies(64, n, k, G) and not fp8_gemm_applies(256, n, k, 64)
    w = cases.layer_weights(n, k, 6)
    codes, xs = _codes(m, k, seed=6)
    wd = cases.on_device(w, device)
    x8 = torch.from_numpy(codes).to(device).view(torch.float8_e4m3fn)
    s = torch.from_numpy(xs).to(device).reshape(m, 1)
    y = torch.ops.tokenforge.w4a8_linear(x8, s, wd.qweight_t, wd.scales, wd.qzeros, None, G, "hip")
    assert torch.equal(y, _run(codes, xs, w, fp8_gemm_config(256, n, k), device))
    _check(y, codes, xs, w, "op")


def test_the_w4a16_entry_rejects_an_fp8_config(device: torch.device) -> None:
    from tokenforge.kernels.hip.w4a16 import w4a16_gemm

    w = cases.on_device(cases.layer_weights(256, 256, 0), device)
    x = torch.zeros((128, 256), dtype=torch.float16, device=device)
    with pytest.raises(ValueError, match="e4m3"):
        w4a16_gemm(x, w.qweight_t, w.scales, w.qzeros, G, FP8_CONFIGS[0])
