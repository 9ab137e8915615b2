"""A decoder-layer stack of the library's ops, captured in one HIP graph: every replay equals
the eager pass bit for bit, with eager work on other inputs between replays (the split-K
reductions are fixed-order and no kernel depends on launch timing).

Layers at the Qwen2.5-7B shapes (qkv 4608x3584 with bias, o_proj, gate_up 37888x3584, down
3584x18944), RMSNorm + FP8 in front of qkv and gate_up, fp16(q * scale) as the linear input
(the torch expression, or the norm's own fp16 output in the fused pass),
attention as the identity on the value slice, SiLU(gate) * up, residual adds. Configs are
the library defaults for each M (the GEMV, register-streamed and pipelined GEMM families).

At full depth (28 layers, M in {1, 2048}), the benchmark's fused pass (each norm inside the
op of the linear it feeds) equals the unfused pass bit for bit and replays to the same bits.
The W4A8 pass (qkv and gate_up on the e4m3 codes) replays to its eager bits, and its
divergence from the fused pass stays within the stack's own sensitivity to one rounding of
its input.
"""

from __future__ import annotations

import pytest
import torch

import tokenforge.kernels.ops  # noqa: F401  (registers torch.ops.tokenforge)
from tokenforge.kernels.autotune import synthetic_layer

pytestmark = pytest.mark.gpu
G = 128
H, QKV, INTER = 3584, 4608, 18944
SHAPES = [(QKV, H), (H, H), (2 * INTER, H), (H, INTER)]


def _layers(device: torch.device, count: int) -> list:  # type: ignore[type-arg]
    out = []
    for li in range(count):
        ws = [synthetic_layer(n, k, G, device, seed=100 * li + i) for i, (n, k) in enumerate(SHAPES)]
        gen = torch.Generator(device=device).manual_seed(7 + li)
        bias = (0.1 * torch.randn((QKV,), generator=gen, device=device)).to(torch.float16)
        g1 = (1 + 0.1 * torch.randn((H,), generator=gen, device=device)).to(torch.float16)
        g2 = (1 + 0.1 * torch.randn((H,), generator=gen, device=device)).to(torch.float16)
        out.append((ws, bias, g1, g2))
    return out


def _norm_to_f16(x: torch.Tensor, gamma: torch.Tensor, fused: bool) -> torch.Tensor:
    """RMSNorm + FP8, then the fp16 linear input fp16(q * scale): from the norm's own second
    output (``fused``) or as the torch expression."""
    ops = torch.ops.tokenforge
    if fused:
        return ops.rmsnorm_fp8_quant_dequant(x, gamma, 1e-6, None)[2]
    q8, s = ops.rmsnorm_fp8_quant(x, gamma, 1e-6, None)
    return (q8.to(torch.float32) * s).to(torch.float16)


def _pass(x: torch.Tensor, layers: list, fused: bool = False) -> torch.Tensor:  # type: ignore[type-arg]
    """One pass; ``fused`` runs the residual adds and SiLU*mul as linear epilogues and takes
    the linear inputs from the norm's fp16 output."""
    ops = torch.ops.tokenforge
    m = x.shape[0]
    for (qkv, o, gu, down), bias, g1, g2 in layers:
        a = _norm_to_f16(x, g1, fused)
        y = ops.w4a16_linear(a, *qkv, bias, G, "hip")
        v = y[:, QKV - 512:].reshape(m, 4, 1, 128)
        attn = v.expand(m, 4, 7, 128).reshape(m, H)
        if fused:
            x = ops.w4a16_linear_residual(attn, *o, None, x, G, "hip")
        else:
            x = x + ops.w4a16_linear(attn, *o, None, G, "hip")
        a = _norm_to_f16(x, g2, fused)
        if fused:
            act = ops.w4a16_linear_silu_mul(a, *gu, None, G, "hip")
            x = ops.w4a16_linear_residual(act, *down, None, x, G, "hip")
        else:
            y = ops.w4a16_linear(a, *gu, None, G, "hip")
            act = torch.nn.functional.silu(y[:, :INTER]) * y[:, INTER:]
            x = x + ops.w4a16_linear(act, *down, None, G, "hip")
    return x


@pytest.mark.parametrize("fused", [False, True], ids=["unfused", "fused"])
@pytest.mark.parametrize("m", [1, 24, 300])
def test_stack_replay_is_bit_identical_to_eager(m: int, fused: bool, device: torch.device) -> None:
    layers = _layers(device, 2)
    gen = torch.Generator(device=device).manual_seed(m)
    x = torch.randn((m, H), generator=gen, device=device).to(torch.float16)
    other = torch.randn((m, H), generator=gen, device=device).to(torch.float16)
    eager = _pass(x, layers, fused)
    assert bool(torch.isfinite(eager).all())
    if fused:  # the fused epilogues and the norm's fp16 output round exactly like the torch glue
        assert torch.equal(eager, _pass(x, layers))

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        _pass(x, layers, fused)  # warm-up on the capture stream
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = _pass(x, layers, fused)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), "graph replay differs from the eager pass"
        _pass(other, layers, fused)  # eager work between replays
        torch.cuda.synchronize()


def _pass_norm_in_linear(x: torch.Tensor, layers: list) -> torch.Tensor:  # type: ignore[type-arg]
    """The benchmark's fused pass: each norm inside the op of the linear it feeds
    (``rmsnorm_fp8_w4a16_linear``: one launch at M <= 4, the norm kernel then the linear
    above), residual adds and SiLU*mul as epilogues."""
    ops = torch.ops.tokenforge
    m = x.shape[0]
    for (qkv, o, gu, down), bias, g1, g2 in layers:
        y = ops.rmsnorm_fp8_w4a16_linear(x, g1, 1e-6, *qkv, bias, G, "hip", "none")
        attn = y[:, QKV - 512:].reshape(m, 4, 1, 128).expand(m, 4, 7, 128).reshape(m, H)
        x = ops.w4a16_linear_residual(attn, *o, None, x, G, "hip")
        act = ops.rmsnorm_fp8_w4a16_linear(x, g2, 1e-6, *gu, None, G, "hip", "silu_mul")
        x = ops.w4a16_linear_residual(act, *down, None, x, G, "hip")
    return x


@pytest.mark.parametrize("m", [1, 2048])
def test_28_layer_stack_fused_equals_unfused_and_replays(m: int, device: torch.device) -> None:
    """BASELINE config 5 at its full depth (28 layers) at the decode and prefill M: the fused
    pass equals the unfused torch composition bit for bit, a graph of it replays to the same
    bits (eager work between replays), and the output is finite."""
    layers = _layers(device, 28)
    gen = torch.Generator(device=device).manual_seed(1000 + m)
    x = torch.randn((m, H), generator=gen, device=device).to(torch.float16)
    ref = _pass(x, layers)
    assert bool(torch.isfinite(ref).all()), "non-finite output"
    assert torch.equal(_pass_norm_in_linear(x, layers), ref), "fused pass differs from the unfused one"
    other = torch.randn((m, H), generator=gen, device=device).to(torch.float16)
    st = torch.cuda.Stream(device)
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        _pass_norm_in_linear(x, layers)  # warm-up on the capture stream
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        out = _pass_norm_in_linear(x, layers)
    for _ in range(2):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), "replay differs from eager"
        _pass_norm_in_linear(other, layers)  # eager work between replays
        torch.cuda.synchronize()


def _pass_w4a8(x: torch.Tensor, layers: list) -> torch.Tensor:  # type: ignore[type-arg]
    """The benchmark's W4A8 pass: qkv and gate_up take the norm's e4m3 codes and row scales
    directly (no fp16(q * scale)); o_proj and down stay W4A16 with the residual epilogue."""
    ops = torch.ops.tokenforge
    m = x.shape[0]
    for (qkv, o, gu, down), bias, g1, g2 in layers:
        q8, s = ops.rmsnorm_fp8_quant(x, g1, 1e-6, None)
        y = ops.w4a8_linear(q8, s, *qkv, bias, G, "hip")
        attn = y[:, QKV - 512:].reshape(m, 4, 1, 128).expand(m, 4, 7, 128).reshape(m, H)
        x = ops.w4a16_linear_residual(attn, *o, None, x, G, "hip")
        q8, s = ops.rmsnorm_fp8_quant(x, g2, 1e-6, None)
        act = ops.w4a8_linear(q8, s, *gu, None, G, "hip", "silu_mul")
        x = ops.w4a16_linear_residual(act, *down, None, x, G, "hip")
    return x


@pytest.mark.parametrize("m", [1, 24, 300])
def test_w4a8_stack_replay_is_bit_identical_to_eager(m: int, device: torch.device) -> None:
    layers = _layers(device, 2)
    gen = torch.Generator(device=device).manual_seed(50 + m)
    x = torch.randn((m, H), generator=gen, device=device).to(torch.float16)
    other = torch.randn((m, H), generator=gen, device=device).to(torch.float16)
    eager = _pass_w4a8(x, layers)
    assert bool(torch.isfinite(eager).all())
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        _pass_w4a8(x, layers)  # warm-up on the capture stream
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = _pass_w4a8(x, layers)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), "graph replay differs from the eager pass"
        _pass_w4a8(other, layers)
        torch.cuda.synchronize()


def _normwise(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.float() - b.float()).abs().max() / b.float().abs().max())


@pytest.mark.parametrize("m", [1, 2048])
def test_w4a8_stack_divergence_is_within_the_stacks_own_rounding_sensitivity(m: int, device: torch.device) -> None:
    """The W4A8 pass is not bit-equal to the fused fp16-input pass (the row scale multiplies
    each row's sum instead of each element, and at prefill M the weights are exact), and after
    28 layers the two differ by 10-20% normwise. That is the stack's own sensitivity, not an
    error of the W4A8 kernels: every sublayer re-quantizes its input to e4m3 (3 mantissa bits),
    so a difference of one rounding in the input moves codes and grows through the layers.
    Bound: at depths 1, 4, 14 and 28 the W4A8 pass stays within 1.5x of the divergence the fused
    pass itself shows when each element of its input moves by half an fp16 ulp (measured
    ratios 0.02-0.85). Each W4A8 linear is held to its own oracle in
    tests/gpu/test_shipped_configs.py (a decoder layer stage by stage)."""
    layers = _layers(device, 28)
    gen = torch.Generator(device=device).manual_seed(700 + m)
    x0 = torch.randn((m, H), generator=gen, device=device).to(torch.float16)
    half_ulp = x0.float().abs() * 2.0**-11
    xp = (x0.float() + half_ulp * torch.sign(torch.randn((m, H), generator=gen, device=device))).to(torch.float16)
    fused, w4a8, pert = x0, x0, xp
    for depth, layer in enumerate(layers, start=1):
        fused = _pass_norm_in_linear(fused, [layer])
        w4a8 = _pass_w4a8(w4a8, [layer])
        pert = _pass_norm_in_linear(pert, [layer])
        if depth in (1, 4, 14, 28):
            assert bool(torch.isfinite(w4a8).all()), f"non-finite W4A8 output at depth {depth}"
            d8, dp = _normwise(w4a8, fused), _normwise(pert, fused)
            assert d8 <= 1.5 * dp, f"depth {depth}: W4A8 diverges by {d8:.3e}, the half-ulp perturbation by {dp:.3e}"
