"""T1: W4A16 HIP kernels vs the oracle's fp64 reference on the fp16-dequantized weights.

Mirrors the reference's tests/numerics/test_w4a16.py: every kernel family and code path,
ragged N, bias, split-K, leading dims, zero rows, misaligned and column-major x, bad
layouts, F1 outliers, Inf/NaN propagation, zero and denormal scales, all-zero weights.
Two bounds are checked on every output: the derived tolerance
``c * sqrt(K) * eps_fp16 * max|x| * max|w|`` (c calibrated against the vendor fp16 GEMM on
this GPU) and the north-star bound ``max|y - ref32| / max|ref32| <= 1e-2`` against an fp32
dequant-then-matmul.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import tokenforge.kernels.ops  # noqa: F401  (registers torch.ops.tokenforge)
from oracle import pack as opack
from oracle import reference as oref
from tests.numerics import cases
from tests.numerics import shapes
from tests.numerics.tolerance import contract
from tokenforge.kernels.config import GemmConfig
from tokenforge.kernels.hip.w4a16 import w4a16_dequant, w4a16_gemm
from tokenforge.kernels.metrics import KERNEL_CALLS
from tokenforge.kernels.pack import W4A16Weights

pytestmark = pytest.mark.gpu
G = cases.GROUP_SIZE


def _linear(x: torch.Tensor, w: W4A16Weights, bias: torch.Tensor | None = None) -> torch.Tensor:
    return torch.ops.tokenforge.w4a16_linear(
        x, w.qweight_t, w.scales, w.qzeros, bias, w.group_size, "hip"
    )


def _assert_close(y: torch.Tensor, x: torch.Tensor, w: opack.W4A16Weights, bias=None) -> None:
    xn = x.detach().cpu().numpy()
    bn = None if bias is None else bias.detach().cpu().numpy()
    ref = oref.w4a16_reference(xn, w, bn)
    y64 = y.detach().cpu().numpy().astype(np.float64)
    w16 = opack.dequantize_tf(w)
    ref32 = xn.astype(np.float32) @ w16.astype(np.float32).T
    if bn is not None:
        ref32 = ref32 + bn.astype(np.float32)
    outcome = contract("cuda").check(y64, ref, ref32, xn, w16)
    assert outcome.ok, str(outcome)


SUITE = shapes.active()
SHAPES = SUITE.shapes


@pytest.mark.parametrize("m", SUITE.m_values)
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{s.model}/{s.layer}" for s in SHAPES])
def test_linear_shape_suite(shape, m: int, device: torch.device) -> None:  # type: ignore[no-untyped-def]
    for seed in cases.TEST_SEEDS:
        w = cases.layer_weights(shape.n, shape.k, seed)
        x = cases.activations(m, shape.k, seed)
        y = _linear(x.to(device), cases.on_device(w, device))
        assert y.shape == (m, shape.n)
        assert y.dtype == torch.float16
        _assert_close(y, x, w)


PATH_CONFIGS = [
    GemmConfig("gemv_dot", 1, 16, 128, 1, 4, 2),
    GemmConfig("gemv_dot", 1, 32, 128, 1, 2, 2),
    GemmConfig("gemv_dot", 2, 16, 128, 1, 2, 2),
    GemmConfig("gemv_dot", 4, 16, 128, 1, 8, 2),
    GemmConfig("gemv_dot", 1, 16, 256, 1, 4, 4),
    GemmConfig("gemv_dot", 4, 16, 256, 1, 8, 4),
    GemmConfig("gemv_mfma", 16, 16, 128, 1, 1, 2),
    GemmConfig("gemv_mfma", 16, 64, 128, 1, 4, 2),
    GemmConfig("gemv_mfma", 16, 32, 128, 1, 8, 4),
    GemmConfig("gemv_mfma", 16, 16, 128, 1, 2, 8),
    GemmConfig("gemv_mfma", 16, 32, 128, 1, 2, 2),
    GemmConfig("gemv_mfma", 16, 16, 128, 1, 8, 2),
    # block_k 256: waves over row tiles (200 rows: the last workgroup's last waves are empty)
    GemmConfig("gemv_mfma", 16, 16, 256, 1, 4, 4),
    GemmConfig("gemv_mfma", 16, 32, 256, 1, 2, 4),
    GemmConfig("gemv_mfma", 16, 16, 256, 1, 8, 4),
    GemmConfig("gemv_mfma", 16, 16, 256, 1, 4, 4),
    GemmConfig("gemv_mfma", 16, 32, 256, 1, 2, 2),
    GemmConfig("gemv_mfma", 16, 16, 128, 1, 1, 2),
    GemmConfig("gemv_mfma", 16, 16, 128, 1, 16, 4),
    GemmConfig("gemv_mfma", 16, 64, 128, 1, 8, 2),
    GemmConfig("gemv_mfma", 16, 64, 128, 1, 2, 2),
    GemmConfig("gemv_mfma", 32, 32, 128, 1, 2, 2),
    GemmConfig("gemv_mfma", 32, 16, 256, 1, 4, 2),
    GemmConfig("gemv_mfma", 16, 32, 256, 1, 8, 4),
    GemmConfig("gemv_mfma", 16, 32, 128, 1, 8, 4),
    GemmConfig("gemv_mfma", 32, 32, 128, 1, 4, 2),
    GemmConfig("gemm_mfma", 64, 64, 64, 1, 4, 2),
    GemmConfig("gemm_mfma", 64, 128, 64, 3, 4, 2),
    GemmConfig("gemm_mfma", 128, 128, 32, 2, 4, 2),
    GemmConfig("gemm_mfma", 256, 128, 64, 4, 4, 2),
    GemmConfig("gemm_mfma", 128, 256, 64, 1, 4, 2),
    # pipelined form: x in three (num_stages 4) or two (3) LDS stages, weights two blocks
    # ahead, 4 or 8 waves; split_k 3 over the 8 K blocks gives slices of 2 and 3 blocks (the
    # odd tail iteration)
    GemmConfig("gemm_mfma", 256, 160, 64, 1, 4, 4),
    GemmConfig("gemm_mfma", 128, 128, 64, 3, 4, 4),
    GemmConfig("gemm_mfma", 64, 256, 64, 2, 4, 4),
    GemmConfig("gemm_mfma", 256, 192, 64, 1, 4, 4),
    GemmConfig("gemm_mfma", 256, 96, 64, 3, 4, 4),
    GemmConfig("gemm_mfma", 128, 192, 64, 1, 4, 4),
    GemmConfig("gemm_mfma", 256, 128, 64, 1, 4, 4),
    GemmConfig("gemm_mfma", 128, 256, 64, 1, 4, 4),
    GemmConfig("gemm_mfma", 256, 256, 64, 1, 8, 3),
    GemmConfig("gemm_mfma", 256, 192, 64, 3, 8, 3),
    GemmConfig("gemm_mfma", 256, 192, 64, 1, 8, 4),
    GemmConfig("gemm_mfma", 256, 128, 64, 2, 8, 3),
    GemmConfig("gemm_mfma", 128, 256, 64, 3, 8, 3),
    GemmConfig("gemm_mfma", 256, 160, 64, 1, 8, 3),
    # skinny form (block_k 128): weights streamed into MFMA registers, x in LDS stages
    GemmConfig("gemm_mfma", 16, 64, 128, 1, 4, 3),
    GemmConfig("gemm_mfma", 32, 128, 128, 3, 4, 3),
    GemmConfig("gemm_mfma", 64, 256, 128, 1, 4, 3),
    GemmConfig("gemm_mfma", 128, 64, 128, 2, 4, 3),
    GemmConfig("gemm_mfma", 64, 128, 128, 1, 4, 2),
    GemmConfig("gemm_mfma", 128, 128, 128, 1, 4, 3),
    # ... with two waves along M
    GemmConfig("gemm_mfma", 256, 160, 128, 1, 4, 2),
    GemmConfig("gemm_mfma", 256, 160, 128, 3, 4, 2),
]


def _m_list(cfg: GemmConfig) -> tuple[int, ...]:
    if cfg.kernel == "gemv_dot":
        return tuple(sorted({1, cfg.block_m}))
    return (1, cfg.block_m - 1, cfg.block_m + 3)


def _cfg_id(c: GemmConfig) -> str:
    return f"{c.kernel}-bm{c.block_m}-bn{c.block_n}-bk{c.block_k}-sk{c.split_k}-w{c.num_warps}-st{c.num_stages}"


@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("cfg", PATH_CONFIGS, ids=_cfg_id)
def test_every_code_path(cfg: GemmConfig, with_bias: bool, device: torch.device) -> None:
    n, k = 200, 512  # N not a multiple of any block_n
    w = cases.layer_weights(n, k, 0)
    b = cases.bias(n, 0) if with_bias else None
    wd = cases.on_device(w, device)
    for m in _m_list(cfg):
        x = cases.activations(m, k, 0)
        y = w4a16_gemm(
            x.to(device), wd.qweight_t, wd.scales, wd.qzeros, G, cfg, None if b is None else b.to(device)
        )
        _assert_close(y, x, w, b)


@pytest.mark.parametrize(
    "cfg",
    [
        GemmConfig("gemv_mfma", 16, 64, 128, 1, 1, 2),
        GemmConfig("gemv_mfma", 16, 32, 128, 1, 1, 4),
        GemmConfig("gemv_mfma", 32, 16, 128, 1, 1, 2),
        GemmConfig("gemv_mfma", 16, 16, 128, 1, 1, 8),
        GemmConfig("gemv_mfma", 16, 16, 256, 1, 2, 8),  # one shared x, partial last step
    ],
    ids=_cfg_id,
)
def test_gemv_staging_windows(cfg: GemmConfig, device: torch.device) -> None:
    """One wave over a long K with group 32: its x slice (up to 32 rows) exceeds the LDS, so
    the wave stages several windows. K = 8288 also ends in a partial 128-wide step (the
    kernels that check each step's bounds per lane). The shared-x form (block_k 256) stages all
    of x once: one row fits, 15 rows do not and the call is rejected before any launch."""
    n, k, group = 200, 8288, 32
    w = cases.layer_weights(n, k, 3, group)
    wd = cases.on_device(w, device)
    for m in _m_list(cfg):
        x = cases.activations(m, k, 3)
        if cfg.block_k == 256 and m > 1:
            with pytest.raises(ValueError, match="fit the device's LDS"):
                w4a16_gemm(x.to(device), wd.qweight_t, wd.scales, wd.qzeros, group, cfg)
            continue
        y = w4a16_gemm(x.to(device), wd.qweight_t, wd.scales, wd.qzeros, group, cfg)
        _assert_close(y, x, w)


@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize(
    "cfg",
    [GemmConfig("gemm_mfma", 16, 64, 128, 1, 4, 3), GemmConfig("gemm_mfma", 64, 128, 128, 3, 4, 2),
     GemmConfig("gemm_mfma", 128, 64, 128, 1, 4, 3), GemmConfig("gemm_mfma", 256, 160, 128, 2, 4, 2)],
    ids=_cfg_id,
)
def test_skinny_gemm_groups_and_partial_k(cfg: GemmConfig, group: int, device: torch.device) -> None:
    """The skinny kernel reads each lane's group itself (any group size); for groups 32 and 64
    K ends in a partial 128-wide step whose chunks past K read as zeros."""
    n, k = 200, {32: 8288, 64: 8256, 128: 8320}[group]
    w = cases.layer_weights(n, k, 4, group)
    wd = cases.on_device(w, device)
    for m in (16, 37, cfg.block_m + 3):
        x = cases.activations(m, k, 4)
        y = w4a16_gemm(x.to(device), wd.qweight_t, wd.scales, wd.qzeros, group, cfg)
        _assert_close(y, x, w)


@pytest.mark.parametrize(
    ("m", "cfg"),
    [
        (32, GemmConfig("gemm_mfma", 32, 128, 128, 1, 4, 2)),
        (32, GemmConfig("gemm_mfma", 32, 128, 128, 8, 4, 3)),
        (256, GemmConfig("gemm_mfma", 32, 64, 128, 8, 4, 3)),
        (256, GemmConfig("gemm_mfma", 256, 160, 128, 1, 4, 2)),
        (256, GemmConfig("gemm_mfma", 256, 192, 64, 1, 8, 3)),
    ],
    ids=lambda v: _cfg_id(v) if isinstance(v, GemmConfig) else f"m{v}",
)
def test_staged_x_waits_at_full_size(m: int, cfg: GemmConfig, device: torch.device) -> None:
    """Regression: the x tile streams into LDS stages and each barrier waits for a counted
    number of later loads; when the compiler moved weight loads above the x loads of a step,
    some workgroups read a stage before it landed (wrong rows, varying run to run). Full
    gate_up width, three runs: bit-identical to each other and close to an fp32 product of
    the exact dequantized weights."""
    from tokenforge.kernels.autotune import synthetic_layer

    n, k = 37888, 3584
    qweight_t, scales, qzeros = synthetic_layer(n, k, G, device, seed=5)
    gen = torch.Generator(device=device).manual_seed(6)
    x = torch.randn((m, k), generator=gen, device=device).to(torch.float16)
    wt = w4a16_dequant(qweight_t, scales, qzeros, G).float().t().contiguous()
    ref = x.float() @ wt
    runs = [w4a16_gemm(x, qweight_t, scales, qzeros, G, cfg) for _ in range(3)]
    for y in runs[1:]:
        assert torch.equal(y, runs[0]), "results differ between runs"
    rel = float((runs[0].float() - ref).abs().max()) / float(ref.abs().max())
    assert rel <= 2e-3, f"max error {rel:.3e} of max |y|"


@pytest.mark.parametrize(
    ("layer", "n", "k"),
    [("qkv", 4608, 3584), ("o", 3584, 3584), ("gate_up", 37888, 3584), ("down", 3584, 18944)],
)
def test_decode_full_size_config3(layer: str, n: int, k: int, device: torch.device) -> None:
    """BASELINE config 3 at full size: M in {1, 2, 4} on every Qwen2.5-7B decoder linear,
    through the op (default configs) and through each GEMV form (K split over the waves, waves
    over row tiles, MFMA), against an fp32 product of the exactly dequantized weights (the
    dequant kernel is bit-exact with the oracle's). The same inputs give the same bits in every
    config of one form on repeated calls."""
    from tokenforge.kernels.autotune import synthetic_layer

    qweight_t, scales, qzeros = synthetic_layer(n, k, G, device, seed=11)
    wt = w4a16_dequant(qweight_t, scales, qzeros, G).float().t().contiguous()
    forms = [GemmConfig("gemv_mfma", 16, 16, 128, 1, 8, 2), GemmConfig("gemv_mfma", 16, 16, 256, 1, 4, 4),
             GemmConfig("gemv_mfma", 16, 16, 128, 1, 8, 4), GemmConfig("gemv_mfma", 16, 16, 256, 1, 4, 2)]
    for m in (1, 2, 4):
        gen = torch.Generator(device=device).manual_seed(m)
        x = torch.randn((m, k), generator=gen, device=device).to(torch.float16)
        ref = x.float() @ wt
        scale = float(ref.abs().max())
        outs = [torch.ops.tokenforge.w4a16_linear(x, qweight_t, scales, qzeros, None, G, "hip")]
        outs += [w4a16_gemm(x, qweight_t, scales, qzeros, G, cfg) for cfg in forms]
        for cfg, y in zip(["op"] + forms, outs):
            rel = float((y.float() - ref).abs().max()) / scale
            assert rel <= 2e-3, f"{layer} m={m} {cfg}: max error {rel:.3e} of max |y|"
        again = w4a16_gemm(x, qweight_t, scales, qzeros, G, forms[1])
        assert torch.equal(again, outs[2])


STREAM_FORMS = [GemmConfig("gemv_mfma", 4, 16, 512, 1, w, p) for p in (2, 4) for w in (4, 8, 16)]
STREAM_FORMS_8 = [GemmConfig("gemv_mfma", 8, 16, 512, 1, w, p) for p in (2, 4) for w in (4, 8, 16)]


@pytest.mark.parametrize("split", [1, 2, 4])
@pytest.mark.parametrize("block_m", [4, 8])
@pytest.mark.parametrize(
    ("layer", "n", "k"),
    [("qkv", 4608, 3584), ("o", 3584, 3584), ("gate_up", 37888, 3584), ("down", 3584, 18944)],
)
def test_stream_form_full_size(layer: str, n: int, k: int, block_m: int, split: int, device: torch.device) -> None:
    """The GEMV stream form (block_k 512) on every Qwen2.5-7B decoder linear: block_m 4 at M in
    {1, 2, 4}, block_m 8 at M in {5, 8}, without and with a K split across workgroups (split_k 2
    and 4: ring depth 2; each workgroup stages one K slice of x, the split-K reduce adds the
    slices): every ring depth and wave count against an fp32 product of the exactly dequantized
    weights, bit-identical on a second call; the residual and SiLU*mul epilogues bit-equal to
    torch applied to its own plain output; the W4A8 form on e4m3-representable x equal to the
    W4A16 result at unit scale. Shapes outside the form (x or its slice too long to stage, as
    on down_proj at M >= 4 without a split, or fewer K steps per slice than waves) are rejected
    before any launch."""
    from dataclasses import replace

    from tokenforge.kernels.autotune import synthetic_layer
    from tokenforge.kernels.config import stream_form_applies
    from tokenforge.kernels.hip.w4a16 import w4a8_gemm_ex, w4a16_gemm_ex

    qweight_t, scales, qzeros = synthetic_layer(n, k, G, device, seed=13)
    wt = w4a16_dequant(qweight_t, scales, qzeros, G).float().t().contiguous()
    forms = [replace(c, split_k=split) for c in (STREAM_FORMS if block_m == 4 else STREAM_FORMS_8)
             if split == 1 or c.num_stages == 2]
    for m in ((1, 2, 4) if block_m == 4 else (5, 8)):
        gen = torch.Generator(device=device).manual_seed(20 + m)
        x = torch.randn((m, k), generator=gen, device=device).to(torch.float16)
        ref = x.float() @ wt
        scale = float(ref.abs().max())
        for cfg in forms:
            print(f"{layer} m={m} {cfg}", flush=True)
            if not stream_form_applies(m, n, k, cfg.num_warps, max_m=block_m, split_k=split):
                with pytest.raises(ValueError, match="stream form"):
                    w4a16_gemm(x, qweight_t, scales, qzeros, G, cfg)
                continue
            y = w4a16_gemm(x, qweight_t, scales, qzeros, G, cfg)
            rel = float((y.float() - ref).abs().max()) / scale
            assert rel <= 2e-3, f"{layer} m={m} {cfg}: max error {rel:.3e} of max |y|"
            assert torch.equal(w4a16_gemm(x, qweight_t, scales, qzeros, G, cfg), y)
            r = torch.randn((m, n), generator=gen, device=device).to(torch.float16)
            fused = w4a16_gemm_ex(x, qweight_t, scales, qzeros, G, cfg, None, "residual", r)
            assert torch.equal(fused, r + y), f"{layer} m={m} {cfg}: residual"
            if n % 32 == 0:
                fused = w4a16_gemm_ex(x, qweight_t, scales, qzeros, G, cfg, None, "silu_mul")
                expect = torch.nn.functional.silu(y[:, : n // 2]) * y[:, n // 2 :]
                assert torch.equal(fused, expect), f"{layer} m={m} {cfg}: silu_mul"
            x8 = x.to(torch.float8_e4m3fn)
            one = torch.ones(1, dtype=torch.float32, device=device)
            y8 = w4a8_gemm_ex(x8, one, qweight_t, scales, qzeros, G, cfg, None)
            assert torch.equal(y8, w4a16_gemm(x8.to(torch.float16), qweight_t, scales, qzeros, G, cfg))


def test_stream_form_falls_back_outside_its_shapes(device: torch.device) -> None:
    """The op keeps the stream form's bucket config only where the form applies: on N % 32 ==
    16 the plain call and its SiLU*mul twin both run the K-split GEMV and agree bit for bit."""
    from tokenforge.kernels import autotune
    from tokenforge.kernels.device import gpu_identity

    n, k = 48, 1024
    w = cases.layer_weights(n, k, 9)
    wd = cases.on_device(w, device)
    gpu = gpu_identity(device)
    autotune.get_cache(gpu).put(1, n, k, G, GemmConfig("gemv_mfma", 4, 16, 512, 1, 8, 2))
    x = cases.activations(1, k, 9).to(device)
    y = torch.ops.tokenforge.w4a16_linear(x, wd.qweight_t, wd.scales, wd.qzeros, None, G, "hip")
    fused = torch.ops.tokenforge.w4a16_linear_silu_mul(x, wd.qweight_t, wd.scales, wd.qzeros, None, G, "hip")
    assert torch.equal(fused, torch.nn.functional.silu(y[:, : n // 2]) * y[:, n // 2 :])
    _assert_close(y, x.cpu(), w)


@pytest.mark.parametrize("group_size", [32, 64])
def test_small_group_sizes(group_size: int, device: torch.device) -> None:
    n, k = 96, 384
    w = cases.layer_weights(n, k, 0, group_size)
    wd = cases.on_device(w, device)
    configs = [
        GemmConfig("gemv_mfma", 16, 16, 128, 1, 2, 2),
        GemmConfig("gemv_mfma", 16, 32, 128, 1, 2, 2),
        GemmConfig("gemm_mfma", 64, 64, 32, 2, 4, 2),
    ]
    if group_size == 64:
        configs.append(GemmConfig("gemm_mfma", 128, 128, 64, 1, 4, 2))
        configs.append(GemmConfig("gemm_mfma", 128, 128, 64, 2, 4, 4))
        configs.append(GemmConfig("gemm_mfma", 256, 128, 64, 2, 8, 3))
    for cfg in configs:
        for m in (1, 5, 40):
            x = cases.activations(m, k, 1)
            y = w4a16_gemm(x.to(device), wd.qweight_t, wd.scales, wd.qzeros, group_size, cfg)
            _assert_close(y, x, w)
    assert torch.equal(
        w4a16_dequant(wd.qweight_t, wd.scales, wd.qzeros, group_size).cpu(),
        torch.from_numpy(opack.dequantize_tf(w)),
    )


def test_dequant_kernel_is_exact(device: torch.device) -> None:
    w = cases.layer_weights(200, 384, 0)
    wd = cases.on_device(w, device)
    out = w4a16_dequant(wd.qweight_t, wd.scales, wd.qzeros, G)
    assert torch.equal(out.cpu(), torch.from_numpy(opack.dequantize_tf(w)))
    op = torch.ops.tokenforge.w4a16_dequant(wd.qweight_t, wd.scales, wd.qzeros, G)
    assert torch.equal(op, out)


def test_large_m_routes_to_gemm(device: torch.device) -> None:
    KERNEL_CALLS.reset()
    w = cases.layer_weights(128, 256, 0)
    x = cases.activations(300, 256, 0)
    y = _linear(x.to(device), cases.on_device(w, device))
    _assert_close(y, x, w)
    assert KERNEL_CALLS.value(kernel="hip_gemm", bucket="512") == 1
    x1 = cases.activations(3, 256, 0)
    _linear(x1.to(device), cases.on_device(w, device))
    assert KERNEL_CALLS.value(kernel="hip_gemv", bucket="4") == 1


def test_leading_dims_and_bias_through_op(device: torch.device) -> None:
    w = cases.layer_weights(64, 256, 0)
    b = cases.bias(64, 0)
    x = cases.activations(6, 256, 0)
    y = _linear(x.reshape(2, 3, 256).to(device), cases.on_device(w, device), b.to(device))
    assert y.shape == (2, 3, 64)
    _assert_close(y.reshape(6, 64), x, w, b)


def test_zero_rows(device: torch.device) -> None:
    w = cases.on_device(cases.layer_weights(64, 256, 0), device)
    y = _linear(torch.empty((0, 256), dtype=torch.float16, device=device), w)
    assert y.shape == (0, 64)


def test_non_contiguous_and_misaligned_inputs_are_handled(device: torch.device) -> None:
    w = cases.layer_weights(64, 256, 0)
    wd = cases.on_device(w, device)
    x = cases.activations(4, 256, 0)
    # Column-major view: the op makes it contiguous along K.
    x_cm = x.t().contiguous().t().to(device)
    assert x_cm.stride(1) != 1
    _assert_close(_linear(x_cm, wd), x, w)
    # Storage offset of one fp16 element: base pointer is not 16-byte aligned.
    buf = torch.empty(4 * 256 + 1, dtype=torch.float16, device=device)
    x_mis = buf[1:].view(4, 256)
    x_mis.copy_(x.to(device))
    assert x_mis.data_ptr() % 16 != 0
    _assert_close(_linear(x_mis, wd), x, w)
    # Row stride that is not a multiple of 8 elements.
    big = torch.zeros((4, 260), dtype=torch.float16, device=device)
    big[:, :256] = x.to(device)
    x_str = big[:, :256]
    assert x_str.stride(0) == 260
    _assert_close(_linear(x_str, wd), x, w)


def test_rejects_bad_weight_layouts(device: torch.device) -> None:
    w = cases.on_device(cases.layer_weights(64, 256, 0), device)
    x = cases.activations(1, 256, 0).to(device)
    cfg = GemmConfig("gemv_mfma", 16, 16, 128, 1, 1, 2)
    with pytest.raises(ValueError, match="contiguous"):
        w4a16_gemm(x, w.qweight_t.t().contiguous().t(), w.scales, w.qzeros, G, cfg)
    with pytest.raises(ValueError, match="encodes K"):
        w4a16_gemm(x[:, :128], w.qweight_t, w.scales, w.qzeros, G, cfg)
    with pytest.raises(TypeError, match="fp16"):
        w4a16_gemm(x.float(), w.qweight_t, w.scales, w.qzeros, G, cfg)
    with pytest.raises(ValueError, match="divide"):
        w4a16_gemm(x, w.qweight_t, w.scales, w.qzeros, G, GemmConfig("gemm_mfma", 64, 64, 256, 1, 4, 2))
    with pytest.raises(ValueError, match="compiled variant"):
        w4a16_gemm(x, w.qweight_t, w.scales, w.qzeros, G, GemmConfig("gemv_mfma", 48, 16, 128, 1, 1, 2))


def test_shared_x_variant_rejects_x_larger_than_the_lds(device: torch.device) -> None:
    """block_k 256 keeps all of x in LDS: 4 rows of K = 32768 (256 KiB) cannot run."""
    w = cases.on_device(cases.layer_weights(16, 32768, 1), device)
    x = cases.activations(4, 32768, 1).to(device)
    with pytest.raises(ValueError, match="fit"):
        w4a16_gemm(x, w.qweight_t, w.scales, w.qzeros, G, GemmConfig("gemv_mfma", 16, 16, 256, 1, 8, 4))
    with pytest.raises(ValueError, match="fit"):
        w4a16_gemm(x, w.qweight_t, w.scales, w.qzeros, G, GemmConfig("gemv_mfma", 16, 16, 256, 1, 4, 2))
    # one row fits (64 KiB)
    for cfg in (GemmConfig("gemv_mfma", 16, 16, 256, 1, 8, 4), GemmConfig("gemv_mfma", 16, 16, 256, 1, 4, 2)):
        y = w4a16_gemm(x[:1].contiguous(), w.qweight_t, w.scales, w.qzeros, G, cfg)
        _assert_close(y, cases.activations(4, 32768, 1)[:1], cases.layer_weights(16, 32768, 1))


def test_cpu_tensors_take_the_torch_route(device: torch.device) -> None:
    """Host tensors follow the reference's torch_reference decision into the torch route (the
    GPU kernels never see them) and meet the same contract as the GPU result; a GPU call never
    falls back to it."""
    w = cases.layer_weights(64, 256, 0)
    wc = cases.on_device(w, torch.device("cpu"))
    x = cases.activations(2, 256, 0)
    y = _linear(x, wc)
    assert y.device.type == "cpu"
    _assert_close(y, x, w)
    y_gpu = _linear(x.to(device), cases.on_device(w, device))
    assert y_gpu.device.type == "cuda"
    _assert_close(y_gpu, x, w)


# ----------------------------------------------------------------------------- F1 and edges


def _weights_from_ints(q: torch.Tensor, z: torch.Tensor, s: torch.Tensor) -> opack.W4A16Weights:
    """q [K, N] ints, z [K//G, N] ints, s [K//G, N] fp16 -> oracle TokenForge weights."""
    qweight, qzeros = opack.awq_pack(q.to(torch.int32).numpy(), z.to(torch.int32).numpy())
    return opack.pack_awq(qweight, qzeros, s.to(torch.float16).numpy(), G)


F1_CONFIGS = (
    GemmConfig("gemv_mfma", 16, 16, 128, 1, 2, 2),
    GemmConfig("gemv_mfma", 16, 16, 128, 1, 2, 2),
    GemmConfig("gemm_mfma", 64, 64, 64, 2, 4, 2),
)


def test_f1_outliers_cancel_without_fp16_overflow(device: torch.device) -> None:
    """Products of 6e4 x 1.6 overflow fp16; fp32 products + accumulation must cancel them."""
    k, n = 256, 64
    gen = torch.Generator().manual_seed(0)
    q = torch.randint(0, 16, (k, n), generator=gen)
    q[1] = q[0] = 15  # rows 0 and 1 share group 0 -> identical dequantized weights
    z = torch.full((k // G, n), 7)
    s = torch.full((k // G, n), 0.2)
    w = _weights_from_ints(q, z, s)
    wd = cases.on_device(w, device)
    x = (torch.randn((2, k), generator=gen) * 0.5).to(torch.float16)
    x[:, 0], x[:, 1] = 6e4, -6e4
    for cfg in F1_CONFIGS:
        y = w4a16_gemm(x.to(device), wd.qweight_t, wd.scales, wd.qzeros, G, cfg)
        assert bool(torch.isfinite(y).all()), f"spurious Inf/NaN with {cfg}"
        assert np.isfinite(oref.w4a16_reference(x.numpy(), w)).all()
        _assert_close(y, x, w)


def test_f1_real_inf_and_nan_propagate(device: torch.device) -> None:
    w = cases.layer_weights(64, 256, 0)
    wd = cases.on_device(w, device)
    x = cases.activations(16, 256, 0)
    x[0, 5] = float("inf")
    x[1, 7] = float("-inf")
    x[2, 9] = float("nan")
    ref16 = torch.from_numpy(oref.w4a16_reference(x.numpy(), w)).to(torch.float16)
    configs = (
        GemmConfig("gemv_mfma", 16, 16, 128, 1, 2, 2),
        GemmConfig("gemv_mfma", 16, 16, 128, 1, 2, 2),
        GemmConfig("gemm_mfma", 64, 64, 64, 2, 4, 2),
    )
    for cfg in configs:
        rows = x[:16]
        y = w4a16_gemm(rows.to(device), wd.qweight_t, wd.scales, wd.qzeros, G, cfg).cpu()
        r = ref16[: rows.shape[0]]
        assert torch.equal(torch.isnan(y), torch.isnan(r)), cfg
        assert torch.equal(torch.isposinf(y), torch.isposinf(r)), cfg
        assert torch.equal(torch.isneginf(y), torch.isneginf(r)), cfg
        assert bool(torch.isfinite(y[3:]).all()), "Inf leaked into clean rows"


@pytest.mark.parametrize("scale_value", [0.0, 2.0**-24, 6e-6])  # zero, min denormal, denormal
def test_zero_and_denormal_scales(scale_value: float, device: torch.device) -> None:
    k, n = 256, 64
    gen = torch.Generator().manual_seed(1)
    q = torch.randint(0, 16, (k, n), generator=gen)
    z = torch.randint(0, 16, (k // G, n), generator=gen)
    s = torch.rand((k // G, n), generator=gen) * 0.01 + 1e-3
    s[0, :] = scale_value  # group 0 of every column
    w = _weights_from_ints(q, z, s)
    wd = cases.on_device(w, device)
    x = cases.activations(3, k, 0)
    for cfg in (GemmConfig("gemv_mfma", 16, 16, 128, 1, 1, 2),) + F1_CONFIGS:
        rows = x[: min(3, cfg.block_m)]
        y = w4a16_gemm(rows.to(device), wd.qweight_t, wd.scales, wd.qzeros, G, cfg)
        assert bool(torch.isfinite(y).all())
        _assert_close(y, rows, w)
    assert torch.equal(
        w4a16_dequant(wd.qweight_t, wd.scales, wd.qzeros, G).cpu(),
        torch.from_numpy(opack.dequantize_tf(w)),
    )


def test_all_zero_weights_are_exact(device: torch.device) -> None:
    k, n = 128, 16
    w = _weights_from_ints(torch.full((k, n), 9), torch.full((1, n), 9), torch.full((1, n), 0.5))
    y = _linear(cases.activations(2, k, 0).to(device), cases.on_device(w, device))
    assert bool((y == 0).all())


# ----------------------------------------------------------------------------- determinism


def test_split_k_is_deterministic_and_graph_safe(device: torch.device) -> None:
    """F5: same inputs and config -> bit-identical output, eager and under HIP-graph replay."""
    w = cases.on_device(cases.layer_weights(1152, 896, 0), device)
    configs = [
        GemmConfig("gemv_mfma", 16, 32, 128, 1, 4, 2),
        GemmConfig("gemv_mfma", 16, 16, 128, 1, 8, 2),
        GemmConfig("gemm_mfma", 64, 64, 64, 7, 4, 2),
    ]
    for cfg in configs:
        m = 1 if cfg is configs[0] else 48
        x = cases.activations(m, 896, 0).to(device)
        first = w4a16_gemm(x, w.qweight_t, w.scales, w.qzeros, G, cfg)
        for _ in range(3):
            assert torch.equal(w4a16_gemm(x, w.qweight_t, w.scales, w.qzeros, G, cfg), first)
        graph = torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            w4a16_gemm(x, w.qweight_t, w.scales, w.qzeros, G, cfg)  # warm the allocator
            with torch.cuda.graph(graph, stream=stream):
                out = w4a16_gemm(x, w.qweight_t, w.scales, w.qzeros, G, cfg)
        torch.cuda.current_stream().wait_stream(stream)
        for _ in range(3):
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, first), cfg
            eager = w4a16_gemm(x, w.qweight_t, w.scales, w.qzeros, G, cfg)
            torch.cuda.synchronize()
            assert torch.equal(eager, first)
