"""The shape table, the tolerance constants and the counters the parity tests rely on."""

from __future__ import annotations

import numpy as np
import pytest

from tests.numerics import shapes
from tests.numerics.calibrate import two_digits_up
from tests.numerics.tolerance import EPS_FP16, contract, half_ulp_fp16, relative_max_error, roundoff_scale
from tokenforge.kernels.metrics import LabeledCounter


def test_qwen_shapes_match_the_model_dimensions() -> None:
    got = {(s.layer, s.n, s.k) for s in shapes.QWEN25_7B.linears()}
    assert got == {
        ("qkv_proj", 4608, 3584), ("o_proj", 3584, 3584),
        ("gate_up_proj", 37888, 3584), ("down_proj", 3584, 18944),
    }
    small = {(s.layer, s.n, s.k) for s in shapes.QWEN25_05B.linears()}
    assert small == {
        ("qkv_proj", 1152, 896), ("o_proj", 896, 896),
        ("gate_up_proj", 9728, 896), ("down_proj", 896, 4864),
    }
    for s in shapes.RAGGED:
        assert s.n % 16 == 8  # a multiple of 8 that no 16-column tile divides


def test_suite_selection(monkeypatch: pytest.MonkeyPatch) -> None:
    monkeypatch.delenv("TOKENFORGE_SHAPE_SUITE", raising=False)
    quick = shapes.active()
    assert quick.name == "quick"
    assert {s.model for s in quick.shapes} == {"qwen2.5-0.5b", "synthetic"}
    assert len(quick.shapes) == 6
    assert quick.m_values == (1, 3, 8, 16, 31, 129)
    monkeypatch.setenv("TOKENFORGE_SHAPE_SUITE", "full")
    full = shapes.active()
    assert {s.model for s in full.shapes} == {"qwen2.5-0.5b", "qwen2.5-7b", "synthetic"}
    assert len(full.shapes) == 10
    assert 256 in full.m_values


def test_error_scale_and_frozen_constants() -> None:
    x = np.array([[1.0, -3.0, 2.0, 0.5]])
    w = np.array([[0.25, -0.5, 0.1, 0.0]])
    assert roundoff_scale(x, w) == pytest.approx(2.0 * EPS_FP16 * 3.0 * 0.5)
    x_inf = np.array([[np.inf, -3.0, 2.0, 0.5]])
    assert roundoff_scale(x_inf, w) == roundoff_scale(x, w)  # non-finite entries are left out
    for dev in ("cpu", "cuda"):
        assert contract(dev).c == 0.13
        assert contract(dev).atol(x, w) == pytest.approx(0.13 * roundoff_scale(x, w))
    with pytest.raises(LookupError, match="calibrate"):
        contract("tpu")


def test_contract_check_measures_both_bounds() -> None:
    x = np.array([[1.0, -3.0, 2.0, 0.5]])
    w = np.array([[0.25, -0.5, 0.1, 0.0], [1.0, 0.0, 0.0, 0.0]])
    ref = x @ w.T
    c = contract("cuda")
    exact = c.check(ref, ref, ref, x, w)
    assert exact.ok and exact.abs_err == 0.0 and exact.normwise == 0.0
    # 2e-3 off an output of 1.0: 2e-3 - 2**-11 above its half ulp, more than the derived bound
    # (~7.6e-4), within 1e-2 normwise
    off = ref + np.array([[0.0, 2e-3]])
    got = c.check(off, ref, ref, x, w)
    assert not got.ok and got.abs_err == pytest.approx(2e-3 - 2.0**-11) and got.normwise < 1e-2
    # the output rounding alone is not counted: half an ulp off passes
    assert c.check(ref + np.array([[0.0, 2.0**-11]]), ref, ref, x, w).ok
    ref_nan = ref.copy()
    ref_nan[0, 1] = np.nan  # a non-finite reference entry takes no part
    assert c.check(off, ref_nan, ref_nan, x, w).ok


def test_normwise_and_rounding_of_c() -> None:
    ref = np.array([1.0, -4.0, np.nan])
    assert relative_max_error(np.array([1.02, -4.0, 0.0]), ref) == pytest.approx(0.02 / 4.0)
    assert two_digits_up(0.1245726352188545) == 0.13
    assert two_digits_up(0.13) == 0.13
    assert two_digits_up(0.0071) == 0.0071
    assert two_digits_up(2.01) == 2.1


def test_labeled_counter() -> None:
    c = LabeledCounter("tokenforge_test_counter", "test", ("kernel", "bucket"))
    c.inc(kernel="hip_gemv", bucket="1")
    c.inc(2.0, kernel="hip_gemv", bucket="1")
    c.inc(kernel="hip_gemm", bucket="256")
    assert c.value(kernel="hip_gemv", bucket="1") == 3.0
    assert c.value(kernel="hip_gemm", bucket="1") == 0.0
    assert c.total() == 4.0
    assert c.snapshot() == {("hip_gemv", "1"): 3.0, ("hip_gemm", "256"): 1.0}
    with pytest.raises(ValueError, match="missing"):
        c.inc(kernel="hip_gemv")
    with pytest.raises(ValueError, match="unexpected"):
        c.value(kernel="hip_gemv", bucket="1", reason="x")
    c.reset()
    assert c.total() == 0.0
    # A second family of the same name (a module imported twice) shares the exporter.
    again = LabeledCounter("tokenforge_test_counter", "test", ("kernel", "bucket"))
    again.inc(kernel="hip_gemv", bucket="1")
    assert again.value(kernel="hip_gemv", bucket="1") == 1.0


def test_half_ulp_is_half_the_fp16_spacing() -> None:
    v = np.array([0.0, 1e-6, 2.0**-14, 0.3, 1.0, 1.999, 2.0, 3.7, 1000.0, -2.5, 60000.0])
    expect = np.spacing(np.abs(v).astype(np.float16)).astype(np.float64) / 2
    # a value just below a power of two has the spacing of its own binade
    expect[5] = 2.0**-11
    np.testing.assert_array_equal(half_ulp_fp16(v), expect)


def test_the_exactly_rounded_product_always_meets_the_bound() -> None:
    """A draw whose largest output (2.1) sits near an fp16 rounding midpoint: the fp64 product
    rounded to fp16 is off by 9.74e-4, above c * roundoff scale (9.36e-4) but within half an
    ulp, so it passes (and so does every kernel whose accumulation error is within the bound)."""
    import oracle.pack as opack
    import oracle.reference as oref
    from tests.numerics import cases

    n, k, m, g, seed = 448, 384, 167, 64, 134
    w = cases.layer_weights(n, k, seed, g)
    x = cases.activations(m, k, seed).numpy()
    b = cases.bias(n, seed).numpy()
    ref = oref.w4a16_reference(x, w, b)
    w16 = opack.dequantize_tf(w)
    rounded = ref.astype(np.float16).astype(np.float64)
    c = contract("cuda")
    assert float(np.abs(rounded - ref).max()) > c.atol(x, w16)  # the old form fails every fp16 kernel
    assert c.check(rounded, ref, ref, x, w16).ok
