"""T1/T2: fused RMSNorm + e4m3 HIP kernel vs the oracle and vs the reference's torch order.

Bars (north star): codes and scales bit-exact against the oracle restatement of
reference.py:35-56 (which forms the fp32 mean from the exact sum, as the kernel does);
against the reference's literal torch order, codes within one e4m3 code on < 0.1% of the
elements, caused only by last-ulp differences of torch's fp32 ``mean``. The reference's own
assertions (every row reaches 448, dequantization within 2^-3, saturation, signed zeros,
MIN_SCALE on a zero row) are kept. The kernel's two forms (a row per workgroup, a row per
wave) are each held to the same bars; "auto" is the form the hot path picks.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import tokenforge.kernels.ops  # noqa: F401
from oracle import reference as oref
from tokenforge.kernels.hip.rmsnorm_fp8 import (
    FP8_E4M3_MAX,
    e4m3_encode,
    rmsnorm_fp8_quant,
    rmsnorm_fp8_quant_dequant,
)

pytestmark = pytest.mark.gpu
EPS = 1e-6
FORMS = ("auto", "row_per_block", "row_per_wave")


def _form_applies(form: str, h: int) -> bool:
    """The row-per-wave form needs 16-byte rows (h % 8 == 0) and h <= 8192."""
    return form != "row_per_wave" or (h % 8 == 0 and h <= 8192)


def _inputs(t: int, h: int, seed: int, scale: float = 2.0) -> tuple[torch.Tensor, torch.Tensor]:
    """The reference test's generator (test_rmsnorm_fp8.py:30-34)."""
    gen = torch.Generator().manual_seed(seed)
    x = (torch.randn((t, h), generator=gen) * scale).to(torch.float16)
    w = (torch.rand((h,), generator=gen) + 0.5).to(torch.float16)
    return x, w


def baseline_inputs(t: int, h: int = 3584, seed: int = 0) -> tuple[torch.Tensor, torch.Tensor, list[int]]:
    """x ~ N(0,1) with 8 fixed outlier channels x20, gamma ~ N(1, 0.1)."""
    chan = torch.randperm(h, generator=torch.Generator().manual_seed(0))[:8].tolist()
    gen = torch.Generator().manual_seed(1000 + seed)
    x = torch.randn((t, h), generator=gen)
    x[:, chan] *= 20.0
    gamma = (1.0 + 0.1 * torch.randn((h,), generator=gen)).to(torch.float16)
    return x.to(torch.float16), gamma, chan


def _codes(q: torch.Tensor) -> np.ndarray:
    return q.cpu().view(torch.uint8).numpy()


def _code_distance(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in e4m3 codes between same-sign values (ordering of the low 7 bits)."""
    a = a.astype(np.int16)
    b = b.astype(np.int16)
    mag_a, mag_b = a & 0x7F, b & 0x7F
    same_sign = ((a & 0x80) == (b & 0x80)) | (mag_a == 0) | (mag_b == 0)
    dist = np.abs(mag_a - mag_b)
    dist[~same_sign] = 255
    return dist


def _check_against_torch_order(q: torch.Tensor, s: torch.Tensor, x: torch.Tensor, w: torch.Tensor) -> None:
    y_t = oref.rmsnorm_torch_order(x.numpy(), w.numpy(), EPS)
    q_t, s_t = oref.fp8_quant_reference(y_t)
    dist = _code_distance(_codes(q), q_t)
    assert int(dist.max()) <= 1, f"max code distance {int(dist.max())}"
    assert float((dist > 0).mean()) < 1e-3, "more than 0.1% of codes differ from the torch order"
    rel = np.abs(s.cpu().numpy() - s_t) / s_t
    assert float(rel.max()) <= 1e-3


@pytest.mark.parametrize(("form", "h", "t"),
                         [(f, h, t) for f in FORMS for h in (896, 3584, 1000, 8192) for t in (1, 7, 33)
                          if _form_applies(f, h)])
def test_dynamic_per_token(t: int, h: int, form: str, device: torch.device) -> None:
    x, w = _inputs(t, h, seed=t * h)
    q, s = rmsnorm_fp8_quant(x.to(device), w.to(device), EPS, form=form)
    q_ref, s_ref = oref.rmsnorm_fp8_reference(x.numpy(), w.numpy(), EPS)
    assert q.dtype == torch.float8_e4m3fn
    assert s.shape == (t, 1)
    assert np.array_equal(_codes(q), q_ref)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    _check_against_torch_order(q, s, x, w)
    # Per-token scaling: every row hits the e4m3 maximum at its absmax.
    assert bool((q.cpu().float().abs().amax(dim=-1) == FP8_E4M3_MAX).all())
    # Dequantized values track the fp16 RMSNorm output to e4m3 precision (3 mantissa bits).
    y = oref.rmsnorm(x.numpy(), w.numpy(), EPS).astype(np.float32)
    deq = q.cpu().float().numpy() * s.cpu().numpy()
    rel = np.abs(deq - y) / np.maximum(np.abs(y), float(s_ref.max()))
    assert float(rel.max()) <= 2.0**-3


def _order_sensitive(t: int, h: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Rows whose fp64 sum of squares depends on the order of the adds (1024^2 and 0.25^2 next
    to tiny squares a long way off, the tiny ones moved from row to row), between N(0, 1) rows."""
    x, w = _inputs(t, h, seed=t + h)
    for r in range(0, t, max(1, t // 64)):
        x[r] = 0
        x[r, r % 8], x[r, 2 + r % 8] = 1024, 0.25
        pos = (h // 2 + 8 * r) % (h - 2)
        x[r, pos] = x[r, pos + 2] = 154 * 2.0**-24
    return x, w


@pytest.mark.parametrize(("form", "t", "h"),
                         [(f, t, h) for f in FORMS for t, h in ((1, 3584), (2047, 3584), (2048, 3584), (64, 4096),
                                                                (3, 1000)) if _form_applies(f, h)])
def test_order_sensitive_rows_in_every_form(t: int, h: int, form: str, device: torch.device) -> None:
    """The sum of squares is added in one fixed order in every form (row per workgroup with four
    waves below 2048 rows and two from 2048 on, row per wave): codes and scales equal the
    oracle's on rows where another order rounds var differently."""
    x, w = _order_sensitive(t, h)
    q, s = rmsnorm_fp8_quant(x.to(device), w.to(device), EPS, form=form)
    q_ref, s_ref = oref.rmsnorm_fp8_reference(x.numpy(), w.numpy(), EPS)
    assert np.array_equal(_codes(q), q_ref)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("form", FORMS)
@pytest.mark.parametrize("t", [1, 16, 512, 4096])
def test_baseline_config2_bit_exact(t: int, form: str, device: torch.device) -> None:
    x, gamma, _ = baseline_inputs(t)
    q, s = rmsnorm_fp8_quant(x.to(device), gamma.to(device), EPS, form=form)
    q_ref, s_ref = oref.rmsnorm_fp8_reference(x.numpy(), gamma.numpy(), EPS)
    assert np.array_equal(_codes(q), q_ref)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    _check_against_torch_order(q, s, x, gamma)


def test_static_scale_saturates_exactly(device: torch.device) -> None:
    x, w = _inputs(16, 896, seed=11, scale=3.0)
    scale = np.array([2e-3], dtype=np.float32)
    q, s_out = rmsnorm_fp8_quant(x.to(device), w.to(device), EPS, torch.from_numpy(scale).to(device))
    q_ref, _ = oref.rmsnorm_fp8_reference(x.numpy(), w.numpy(), EPS, scale)
    assert torch.equal(s_out.cpu(), torch.from_numpy(scale))
    y = oref.rmsnorm(x.numpy(), w.numpy(), EPS).astype(np.float32) / scale
    saturated = np.abs(y) >= FP8_E4M3_MAX
    assert int(saturated.sum()) > 100, "test must exercise saturation"
    qf = q.cpu().float().numpy()
    assert np.array_equal(_codes(q), q_ref)
    assert bool((np.abs(qf[saturated]) == FP8_E4M3_MAX).all())
    assert not bool(np.isnan(qf).any()), "saturating cast must never emit NaN"


def test_e4m3_rounding_is_bit_exact_at_every_midpoint(device: torch.device) -> None:
    """Every e4m3 value, every midpoint between neighbours, and the fp32 values either side
    of each midpoint round exactly like PyTorch's ``to(float8_e4m3fn)``, signs included."""
    values = torch.arange(0, 0x7F, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    mids = (values[1:] + values[:-1]) / 2
    up, down = torch.tensor(1e9), torch.tensor(-1e9)
    probe = torch.cat([values, mids, mids.nextafter(up), mids.nextafter(down)])
    probe = torch.cat([probe, -probe, torch.tensor([0.0, -0.0, float("nan"), -float("nan")])])
    gen = torch.Generator().manual_seed(5)
    probe = torch.cat([probe, (torch.rand(1 << 20, generator=gen) * 2 - 1) * 448,
                       (torch.rand(1 << 18, generator=gen) * 2 - 1) * 0.03])
    out = e4m3_encode(probe.to(device))
    assert np.array_equal(_codes(out), probe.to(torch.float8_e4m3fn).view(torch.uint8).numpy())


def _assert_codes_match_nan_aware(codes: np.ndarray, ref: np.ndarray) -> None:
    """Bit-exact, except that a NaN code (0x7F / 0xFF) matches either NaN code: the sign of a
    NaN that an invalid operation creates (0/0, inf*0) is the hardware's default NaN, which
    is negative on x86 (the oracle) and positive on the GPU."""
    nan_k, nan_r = (codes & 0x7F) == 0x7F, (ref & 0x7F) == 0x7F
    assert np.array_equal(nan_k, nan_r), "NaN positions differ"
    assert np.array_equal(codes[~nan_k], ref[~nan_r])


@pytest.mark.parametrize(("t", "h"), [(2050, 3584), (4099, 896), (4100, 8192), (5000, 3584)])
def test_row_per_wave_long_and_ragged_batches(t: int, h: int, device: torch.device) -> None:
    """The row-per-wave form at long batches whose row count leaves the last workgroup with
    fewer than four rows: every code, scale and fp16 output bit-exact."""
    x, gamma, _ = baseline_inputs(t, h, seed=t)
    q, s = rmsnorm_fp8_quant(x.to(device), gamma.to(device), EPS, form="row_per_wave")
    q_ref, s_ref = oref.rmsnorm_fp8_reference(x.numpy(), gamma.numpy(), EPS)
    assert np.array_equal(_codes(q), q_ref)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    qd, sd, a = rmsnorm_fp8_quant_dequant(x.to(device), gamma.to(device), EPS, form="row_per_wave")
    assert np.array_equal(_codes(qd), q_ref)
    assert torch.equal(sd, s)
    _assert_f16_match_nan_aware(a, (qd.to(torch.float32) * sd).to(torch.float16))


@pytest.mark.parametrize("form", FORMS[1:])
def test_special_values_rows_and_scales(form: str, device: torch.device) -> None:
    """Rows with +inf, NaN, an fp16 overflow of y, zeros and -inf (dynamic scale), and static
    scales 0, inf, NaN, negative and tiny: the kernel's exact-rounding slow path."""
    h = 896
    gen = torch.Generator().manual_seed(21)
    x = (torch.randn((6, h), generator=gen) * 2).to(torch.float16)
    w = (torch.rand((h,), generator=gen) + 0.5).to(torch.float16)
    w[5] = 4000.0  # x[2, 5] * rstd * 4000 overflows fp16
    x[0, 3] = float("inf")
    x[1, 7] = float("nan")
    x[2, 5] = 1000.0
    x[3] = 0.0
    x[5, 9] = float("-inf")
    with np.errstate(all="ignore"):
        q_ref, s_ref = oref.rmsnorm_fp8_reference(x.numpy(), w.numpy(), EPS)
    q, s = rmsnorm_fp8_quant(x.to(device), w.to(device), EPS, form=form)
    _assert_codes_match_nan_aware(_codes(q), q_ref)
    s_k = s.cpu().numpy()
    assert np.array_equal(np.isnan(s_k), np.isnan(s_ref))
    assert np.array_equal(s_k[~np.isnan(s_k)].view(np.uint32), s_ref[~np.isnan(s_ref)].view(np.uint32))
    for sc in (0.0, float("inf"), float("nan"), -2e-3, 1e-30):
        scale = np.array([sc], dtype=np.float32)
        with np.errstate(all="ignore"):
            q_ref, _ = oref.rmsnorm_fp8_reference(x.numpy(), w.numpy(), EPS, scale)
        q, _ = rmsnorm_fp8_quant(x.to(device), w.to(device), EPS, torch.from_numpy(scale).to(device), form=form)
        _assert_codes_match_nan_aware(_codes(q), q_ref)


@pytest.mark.parametrize("form", FORMS[1:])
@pytest.mark.parametrize("eps", [0.0, -1.0])
def test_rows_with_infinite_or_nan_rstd(eps: float, form: str, device: torch.device) -> None:
    """eps = 0 on an all-zero row makes rstd = inf (every y = 0 * inf = NaN); eps = -1 makes it
    NaN on rows whose mean square is below 1. H = 896 leaves the last 8-element chunks of every
    thread past the row, which load zeros: their y must not change the row's absmax (the
    vector path takes the max of all chunks without a mask)."""
    h = 896
    gen = torch.Generator().manual_seed(31)
    x = (torch.randn((4, h), generator=gen) * 0.5).to(torch.float16)
    w = (torch.rand((h,), generator=gen) + 0.5).to(torch.float16)
    x[1] = 0.0
    x[3] = (torch.randn((h,), generator=gen) * 3).to(torch.float16)
    with np.errstate(all="ignore"):
        q_ref, s_ref = oref.rmsnorm_fp8_reference(x.numpy(), w.numpy(), eps)
    q, s = rmsnorm_fp8_quant(x.to(device), w.to(device), eps, form=form)
    _assert_codes_match_nan_aware(_codes(q), q_ref)
    s_k = s.cpu().numpy()
    assert np.array_equal(np.isnan(s_k), np.isnan(s_ref))
    assert np.array_equal(s_k[~np.isnan(s_k)].view(np.uint32), s_ref[~np.isnan(s_ref)].view(np.uint32))


def _assert_f16_match_nan_aware(a: torch.Tensor, b: torch.Tensor) -> None:
    an, bn = torch.isnan(a), torch.isnan(b)
    assert torch.equal(an, bn)
    assert torch.equal(a[~an].view(torch.int16), b[~bn].view(torch.int16))


@pytest.mark.parametrize(("form", "t", "h", "aligned"),
                         [(f, t, h, a) for f in FORMS for t, h, a in ((1, 3584, True), (7, 896, True), (33, 3584, True),
                                                                       (5, 1000, False)) if a or f != "row_per_wave"])
def test_dequantized_output_equals_the_torch_expression(t: int, h: int, aligned: bool, form: str,
                                                        device: torch.device) -> None:
    """rmsnorm_fp8_quant_dequant: the codes and scales are rmsnorm_fp8_quant's, bit for bit, and
    the fp16 output is `(q.to(float32) * scale).to(float16)` bit for bit (dynamic and static
    scales, the large one leaving mostly subnormal and zero codes; the scalar path for an
    unaligned x)."""
    x, w = baseline_inputs(t, h, seed=5)[:2] if h == 3584 else _inputs(t, h, seed=5)
    xd = x.to(device)
    if not aligned:
        buf = torch.empty(t * (h + 3) + 1, dtype=torch.float16, device=device)
        xd = buf[1:].view(t, h + 3)[:, :h]
        xd.copy_(x.to(device))
    wd = w.to(device)
    for sc in (None, torch.full((1,), 0.05, device=device), torch.full((1,), 400.0, device=device)):
        q, s, a = rmsnorm_fp8_quant_dequant(xd, wd, EPS, sc, form=form)
        q0, s0 = rmsnorm_fp8_quant(xd, wd, EPS, sc, form="row_per_block")
        assert np.array_equal(_codes(q), _codes(q0))
        assert torch.equal(s, s0)
        _assert_f16_match_nan_aware(a, (q.to(torch.float32) * s).to(torch.float16))


def test_dequantized_output_of_special_rows(device: torch.device) -> None:
    """Rows with inf, NaN and zeros (the kernel's NaN-preserving slow path) and the op's leading dims."""
    h = 896
    gen = torch.Generator().manual_seed(23)
    x = (torch.randn((6, h), generator=gen) * 2).to(torch.float16)
    w = (torch.rand((h,), generator=gen) + 0.5).to(torch.float16)
    x[0, 3] = float("inf")
    x[1, 7] = float("nan")
    x[3] = 0.0
    x[5, 9] = float("-inf")
    q, s, a = torch.ops.tokenforge.rmsnorm_fp8_quant_dequant(x.reshape(2, 3, h).to(device), w.to(device), EPS, None)
    assert q.shape == a.shape == (2, 3, h) and s.shape == (2, 3, 1)
    q0, s0 = rmsnorm_fp8_quant(x.to(device), w.to(device), EPS)
    assert np.array_equal(_codes(q.reshape(6, h)), _codes(q0))
    _assert_f16_match_nan_aware(a.reshape(6, h), (q0.to(torch.float32) * s0).to(torch.float16))


@pytest.mark.parametrize("static", [False, True])
def test_zero_tokens(static: bool, device: torch.device) -> None:
    """T = 0: empty codes and fp16 output, no launch; the dynamic scale is [0, 1], a static
    scale comes back as given."""
    x = torch.empty((0, 896), dtype=torch.float16, device=device)
    w = torch.ones(896, dtype=torch.float16, device=device)
    sc = torch.full((1,), 0.25, device=device) if static else None
    q, s, a = rmsnorm_fp8_quant_dequant(x, w, EPS, sc)
    assert q.shape == a.shape == (0, 896) and q.dtype == torch.float8_e4m3fn and a.dtype == torch.float16
    assert s.shape == ((1,) if static else (0, 1))
    q, s, a = torch.ops.tokenforge.rmsnorm_fp8_quant_dequant(x.reshape(0, 1, 896), w, EPS, sc)
    assert q.shape == a.shape == (0, 1, 896)


def test_zero_row_uses_min_scale(device: torch.device) -> None:
    x = torch.zeros((2, 256), dtype=torch.float16)
    w = torch.ones(256, dtype=torch.float16)
    q, s = rmsnorm_fp8_quant(x.to(device), w.to(device), EPS)
    assert bool((q.cpu().float() == 0).all())
    assert np.array_equal(s.cpu().numpy(), np.full((2, 1), np.float32(oref.MIN_SCALE)))


def test_op_matches_kernel_and_keeps_leading_dims(device: torch.device) -> None:
    x, w = _inputs(6, 896, seed=3)
    q, s = torch.ops.tokenforge.rmsnorm_fp8_quant(x.reshape(2, 3, 896).to(device), w.to(device), EPS, None)
    assert q.shape == (2, 3, 896)
    assert s.shape == (2, 3, 1)
    qk, sk = rmsnorm_fp8_quant(x.to(device), w.to(device), EPS)
    assert np.array_equal(_codes(q.reshape(6, 896)), _codes(qk))
    assert torch.equal(s.reshape(6, 1).cpu(), sk.cpu())


def test_unaligned_rows_take_the_scalar_path(device: torch.device) -> None:
    x, w = _inputs(5, 1000, seed=9)
    buf = torch.empty(5 * 1003 + 1, dtype=torch.float16, device=device)
    xs = buf[1:].view(5, 1003)[:, :1000]
    xs.copy_(x.to(device))
    q, s = rmsnorm_fp8_quant(xs, w.to(device), EPS)
    q_ref, s_ref = oref.rmsnorm_fp8_reference(x.numpy(), w.numpy(), EPS)
    assert np.array_equal(_codes(q), q_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref)


def test_rejects_bad_inputs(device: torch.device) -> None:
    x, w = _inputs(2, 128, seed=0)
    with pytest.raises(ValueError, match="2-D"):
        rmsnorm_fp8_quant(x.reshape(-1).to(device), w.to(device), EPS)
    with pytest.raises(ValueError, match="weight shape"):
        rmsnorm_fp8_quant(x.to(device), w[:64].to(device), EPS)
    with pytest.raises(ValueError, match="single fp32"):
        rmsnorm_fp8_quant(x.to(device), w.to(device), EPS, torch.ones(2, device=device))
