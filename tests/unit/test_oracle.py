"""Pins of the oracle's floating-point functions (oracle/reference.py) on CPU.

Each check is chosen so that a plausible mistake (a dropped term, a wrong rounding, a lost
sign, a transposed operand) fails: library routines (torch's fp8 cast, torch's fp32 mean),
exact rational arithmetic, closed forms.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import pack as P
from oracle import reference as R
from tests.numerics import cases
from tests.numerics.tolerance import contract


def _midpoint_probe() -> torch.Tensor:
    values = torch.arange(0, 0x7F, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    mids = (values[1:] + values[:-1]) / 2
    up, down = torch.tensor(1e9), torch.tensor(-1e9)
    probe = torch.cat([values, mids, mids.nextafter(up), mids.nextafter(down)])
    return torch.cat([probe, -probe, torch.tensor([0.0, -0.0])])


def test_e4m3_encoder_matches_torch_cast_everywhere() -> None:
    gen = torch.Generator().manual_seed(0)
    probe = torch.cat([
        _midpoint_probe(),
        (torch.rand(500_000, generator=gen) * 2 - 1) * 448,
        (torch.rand(200_000, generator=gen) * 2 - 1) * 2.0**-5,
        torch.tensor([448.0, -448.0, 2.0**-6, 2.0**-9, 2.0**-10, 3 * 2.0**-11, 2.0**-6 - 2.0**-10]),
    ])
    expected = probe.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(R.e4m3_encode(probe.numpy()), expected)


def test_e4m3_known_codes_and_nan() -> None:
    pairs = [(0.0, 0x00), (-0.0, 0x80), (448.0, 0x7E), (-448.0, 0xFE), (2.0**-6, 0x08),
             (2.0**-9, 0x01), (2.0**-10, 0x00), (1.5 * 2.0**-9, 0x02), (1.0, 0x38),
             (1.0625, 0x38), (1.1875, 0x3A)]
    got = R.e4m3_encode(np.array([v for v, _ in pairs], dtype=np.float32))
    assert [int(v) for v in got] == [c for _, c in pairs]
    assert int(R.e4m3_encode(np.array([np.nan], dtype=np.float32))[0]) & 0x7F == 0x7F


def test_e4m3_decode_inverts_encode_on_all_codes() -> None:
    codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], dtype=np.uint8)
    assert np.array_equal(R.e4m3_encode(R.e4m3_decode(codes)), codes)
    torch_vals = torch.from_numpy(np.arange(256, dtype=np.uint8)).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(R.e4m3_decode(np.arange(256, dtype=np.uint8)), torch_vals, equal_nan=True)


def test_rmsnorm_constant_row_closed_form() -> None:
    """x = c on every channel: var = c^2, so y = fp16(c / sqrt(c^2 + eps)) * w."""
    h = 1000
    for c in (0.5, -3.0, 1.0):
        x = np.full((1, h), c, dtype=np.float16)
        w = np.full(h, 2.0, dtype=np.float16)
        rstd = np.float32(1) / np.sqrt(np.float32(c * c) + np.float32(1e-6))
        expect = np.float16(np.float32(c) * rstd) * np.float16(2.0)
        assert np.all(R.rmsnorm(x, w, 1e-6) == expect)


def test_rmsnorm_agrees_with_torch_order() -> None:
    """The exact-sum oracle and reference.py's torch fp32 mean differ only by last-ulp var
    differences: identical on almost every element, never more than one fp16 ulp."""
    gen = torch.Generator().manual_seed(1)
    x = (torch.randn((256, 3584), generator=gen) * 2).half().numpy()
    w = (torch.rand(3584, generator=gen) + 0.5).half().numpy()
    a = R.rmsnorm(x, w, 1e-6).astype(np.float32)
    b = R.rmsnorm_torch_order(x, w, 1e-6).astype(np.float32)
    diff = a != b
    assert diff.mean() < 1e-4
    ulp = np.abs(np.spacing(b.astype(np.float16)).astype(np.float32))
    assert bool((np.abs(a - b)[diff] <= ulp[diff] * 1.0001).all())


def test_fp8_quant_dynamic_and_static_semantics() -> None:
    y = np.array([[1.0, -2.0, 0.5, 448.0 * 3], [0.0, 0.0, 0.0, 0.0]], dtype=np.float16)
    q, s = R.fp8_quant_reference(y)
    assert s[0, 0] == np.float32(np.float32(1344.0) / np.float32(448.0))
    assert s[1, 0] == np.float32(R.MIN_SCALE)
    assert int(q[0, 3]) == 0x7E and int(q[1, 0]) == 0
    qs, ss = R.fp8_quant_reference(y, np.array([1e-3], dtype=np.float32))
    assert int(qs[0, 3]) == 0x7E and int(qs[0, 1]) == 0xFE  # saturated, signs kept
    nan_row = np.array([[1.0, np.nan]], dtype=np.float16)
    qn, sn = R.fp8_quant_reference(nan_row)
    assert np.isnan(sn[0, 0]) and (qn[0] & 0x7F == 0x7F).all()


def test_w4a16_reference_exact_on_tiny_inputs() -> None:
    """fp64 reference vs exact rational arithmetic on the fp16-dequantized weights."""
    w = cases.layer_weights(8, 128, 0)
    x = cases.activations(2, 128, 0).numpy()
    b = cases.bias(8, 0).numpy()
    w16 = P.dequantize_tf(w)
    ref = R.w4a16_reference(x, w, b)
    for m in range(2):
        for n in range(8):
            exact = sum(Fraction(float(x[m, k])) * Fraction(float(w16[n, k])) for k in range(128))
            exact += Fraction(float(b[n]))
            assert abs(float(exact) - ref[m, n]) <= 1e-12 * max(1.0, abs(float(exact)))


def test_w4a16_reference_orientation() -> None:
    """A single non-zero weight at (n, k) routes x[:, k] to output column n only."""
    k, n = 128, 16
    q = np.full((k, n), 7, dtype=np.int32)
    q[37, 5] = 9
    qweight, qzeros = P.awq_pack(q, np.full((1, n), 7, dtype=np.int32))
    w = P.pack_awq(qweight, qzeros, np.full((1, n), 0.5, dtype=np.float16), 128)
    x = np.zeros((1, k), dtype=np.float16)
    x[0, 37] = 3.0
    y = R.w4a16_reference(x, w)
    assert y[0, 5] == 3.0 and np.count_nonzero(y) == 1


def test_w4a16_reference_inf_nan_semantics() -> None:
    w = cases.layer_weights(16, 128, 0)
    x = np.zeros((2, 128), dtype=np.float16)
    x[0, 3] = np.inf
    x[1, 4] = np.nan
    y = R.w4a16_reference(x, w)
    w16 = P.dequantize_tf(w).astype(np.float64)
    assert np.array_equal(np.isnan(y[0]), w16[:, 3] == 0)
    assert np.array_equal(np.isposinf(y[0]), w16[:, 3] > 0)
    assert np.isnan(y[1]).all()


def test_fp32_cpu_path_within_derived_tolerance() -> None:
    """reference.py's fp32 CPU path (the timed CPU baseline) meets the CPU tolerance."""
    for n, k in [(200, 256), (1152, 896)]:
        w = cases.layer_weights(n, k, 0)
        x = cases.activations(3, k, 0).numpy()
        y = R.w4a16_fp32(x, w).astype(np.float64)
        ref = R.w4a16_reference(x, w)
        assert float(np.abs(y - ref).max()) <= contract("cpu").atol(x, P.dequantize_tf(w))


@pytest.mark.parametrize("group", [32, 64, 128])
def test_dequant_matches_scalar_fp16(group: int) -> None:
    w = cases.layer_weights(16, 256, 2, group)
    deq = P.dequantize_tf(w)
    q = P.unpack_int4(w.qweight_t)
    z = P.unpack_int4(w.qzeros)
    for nn in (0, 9, 15):
        for kk in (0, group - 1, group, 255):
            g = kk // group
            expect = np.float16(float(q[nn, kk] - z[g, nn])) * w.scales[g, nn]
            assert deq[nn, kk] == expect


def test_w4a8_reference_exact_on_tiny_inputs() -> None:
    """Exact rational arithmetic: y = s_m * sum_k e4m3(c[m, k]) * w[n, k] + b[n]."""
    w = cases.layer_weights(16, 128, 7)
    gen = np.random.default_rng(3)
    codes = gen.integers(0, 256, size=(3, 128), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x38  # no NaN codes: 1.0 instead
    xs = np.array([0.5, 3.0, 2.0**-7], dtype=np.float32)
    b = cases.bias(16, 1).numpy()
    y = R.w4a8_reference(codes, xs, w, b)
    wd = P.dequantize_tf(w)
    for m in range(3):
        for n in (0, 7, 15):
            acc = sum(Fraction(float(R.e4m3_decode(codes[m, k]))) * Fraction(float(wd[n, k])) for k in range(128))
            exact = Fraction(float(xs[m])) * acc + Fraction(float(b[n]))
            assert float(exact) == pytest.approx(y[m, n], rel=1e-12, abs=1e-12)


def test_w4a8_reference_reduces_to_w4a16_and_is_linear_in_scale() -> None:
    w = cases.layer_weights(32, 256, 8)
    codes = np.random.default_rng(4).integers(0, 0x7F, size=(4, 256), dtype=np.uint8)
    one = R.w4a8_reference(codes, np.ones(1, dtype=np.float32), w)
    assert np.array_equal(one, R.w4a16_reference(R.e4m3_decode(codes), w))
    per_row = R.w4a8_reference(codes, np.array([2.0, 4.0, 0.25, 1.0], dtype=np.float32), w)
    assert np.array_equal(per_row, one * np.array([2.0, 4.0, 0.25, 1.0])[:, None])


def test_w4a8_exact_reference_exact_on_tiny_inputs() -> None:
    """fp64 exact-weight W4A8 vs rational arithmetic: (q - z) * s from the integer nibbles and
    the fp16 scales, never rounded."""
    w = cases.layer_weights(8, 256, 1)
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 256, (2, 256)).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x38  # finite codes only
    xs = np.array([0.5, 3.0], dtype=np.float32)
    b = cases.bias(8, 1).numpy()
    y = R.w4a8_exact_reference(codes, xs, w, b)
    q = P.unpack_int4(w.qweight_t)
    z = P.unpack_int4(w.qzeros)
    for m in range(2):
        for n in range(8):
            acc = Fraction(0)
            for k in range(256):
                grp = k // w.group_size
                wk = (int(q[n, k]) - int(z[grp, n])) * Fraction(float(w.scales[grp, n]))
                acc += Fraction(float(R.e4m3_decode(codes[m, k]))) * wk
            exact = acc * Fraction(float(xs[m])) + Fraction(float(b[n]))
            assert abs(float(exact) - y[m, n]) <= 1e-12 * max(1.0, abs(float(exact)))


def test_w4a8_exact_reference_differs_from_the_fp16_weight_form_by_the_weight_rounding() -> None:
    """Against w4a8_reference (weights rounded to fp16 first) the difference is at most the
    fp16 rounding of each weight, half an ulp: |dy| <= sum_k |x_k| * ulp(|w_k|) / 2."""
    w = cases.layer_weights(64, 512, 2)
    rng = np.random.default_rng(6)
    codes = rng.integers(0, 0x7F, (3, 512)).astype(np.uint8)
    xs = np.ones(1, dtype=np.float32)
    exact = R.w4a8_exact_reference(codes, xs, w)
    rounded = R.w4a8_reference(codes, xs, w)
    w16 = np.abs(P.dequantize_tf(w).astype(np.float64))
    bound = np.abs(R.e4m3_decode(codes).astype(np.float64)) @ (np.spacing(w16.astype(np.float16)).astype(np.float64) / 2).T
    assert np.all(np.abs(exact - rounded) <= bound + 1e-12)
    assert np.abs(exact - rounded).max() > 0  # the two forms are not the same function


def _tree_sum_scalar(values: list[float]) -> float:
    """The norm's sum order restated with Python floats (fp64): chunks of 8 zero-padded, each as
    ((e0 + e1) + (e2 + e3)) + ((e4 + e5) + (e6 + e7)), then the chunk sums pairwise (recursive
    halves of a power-of-two count, zero-padded)."""
    sq = [float(v) * float(v) for v in values]
    sq += [0.0] * ((-len(sq)) % 8)
    chunks = []
    for i in range(0, len(sq), 8):
        e = sq[i:i + 8]
        chunks.append(((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7])))
    width = 1
    while width < len(chunks):
        width *= 2
    chunks += [0.0] * (width - len(chunks))

    def pairwise(lo: int, n: int) -> float:
        return chunks[lo] if n == 1 else pairwise(lo, n // 2) + pairwise(lo + n // 2, n // 2)

    return pairwise(0, width)


def test_sum_squares_order_against_a_scalar_restatement() -> None:
    """Bit for bit with an independent scalar restatement of the order, on rows with a wide
    dynamic range (where the order changes the fp64 sum), every length 1..70 and 3584."""
    rng = np.random.default_rng(7)
    for h in list(range(1, 71)) + [3584]:
        mags = rng.choice([2.0**-20, 2.0**-8, 1.0, 2.0**6, 2.0**12], size=(3, h))
        x = (rng.standard_normal((3, h)) * mags).astype(np.float16)
        got = R.sum_squares(x)[:, 0]
        for r in range(3):
            assert got[r] == _tree_sum_scalar(list(x[r])), (h, r)


def test_sum_squares_fixed_order_is_not_any_order() -> None:
    """A row where the fp64 sum depends on the order (1024^2 next to tiny squares): the fixed
    order gives one value, a left-to-right sum another, so a kernel adding in another order is
    caught; the fixed-order sum is within its rounding bound of the exact rational sum."""
    import fractions

    row = np.zeros(3584, dtype=np.float16)
    row[0], row[2] = 1024, 0.25
    row[3584 // 2] = row[3584 // 2 + 2] = np.float16(154 * 2.0**-24)
    for v in range(5, 3584, 97):
        row[v] = np.float16(2.0**-12)
    got = float(R.sum_squares(row[None])[0, 0])
    seq = 0.0
    for v in row:
        seq += float(v) * float(v)
    assert got != seq
    exact = sum(fractions.Fraction(float(v)) ** 2 for v in row)
    assert abs(fractions.Fraction(got) - exact) <= exact * 12 * fractions.Fraction(2) ** -53
