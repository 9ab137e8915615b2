"""T0: op registration is torch.compile- and fake-tensor-safe (test_ops.py in the reference).

Fake-tensor shape propagation runs on CPU; opcheck and torch.compile here execute the real op
on GPU tensors, that is the HIP kernels (tests/unit/test_host_route.py runs the same checks on
host tensors, through the ops' torch route).
"""

from __future__ import annotations

import pytest
import torch
from torch.library import opcheck

import tokenforge.kernels.ops  # noqa: F401
from tests.numerics import cases
from tokenforge.kernels.metrics import KERNEL_CALLS

G = cases.GROUP_SIZE
OPCHECK_TESTS = ("test_schema", "test_faketensor", "test_aot_dispatch_dynamic")


def _layer(device: torch.device, n: int = 64, k: int = 256):  # type: ignore[no-untyped-def]
    w = cases.on_device(cases.layer_weights(n, k, 0), device)
    return w.qweight_t, w.scales, w.qzeros


def test_fake_tensor_shapes() -> None:
    from torch._subclasses.fake_tensor import FakeTensorMode

    qw, s, z = _layer(torch.device("cpu"))
    with FakeTensorMode() as mode:
        x = mode.from_tensor(cases.activations(2, 256, 0)).reshape(1, 2, 256)
        out = torch.ops.tokenforge.w4a16_linear(
            x, mode.from_tensor(qw), mode.from_tensor(s), mode.from_tensor(z), None, G, "hip"
        )
        assert out.shape == (1, 2, 64)
        assert out.dtype == torch.float16
        deq = torch.ops.tokenforge.w4a16_dequant(mode.from_tensor(qw), mode.from_tensor(s), mode.from_tensor(z), G)
        assert deq.shape == (64, 256) and deq.dtype == torch.float16
        xr = mode.from_tensor(cases.activations(6, 256, 1)).reshape(2, 3, 256)
        q, sc = torch.ops.tokenforge.rmsnorm_fp8_quant(xr, mode.from_tensor(torch.ones(256, dtype=torch.float16)), 1e-6, None)
        assert q.shape == (2, 3, 256) and q.dtype == torch.float8_e4m3fn
        assert sc.shape == (2, 3, 1) and sc.dtype == torch.float32


def test_fake_tensor_shapes_of_the_added_ops() -> None:
    """The fused-epilogue and W4A8 ops (no counterpart in the reference) propagate shapes too."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    qw, s, z = _layer(torch.device("cpu"))
    with FakeTensorMode() as mode:
        f = mode.from_tensor
        x = f(cases.activations(6, 256, 0)).reshape(2, 3, 256)
        r = f(torch.zeros((2, 3, 64), dtype=torch.float16))
        out = torch.ops.tokenforge.w4a16_linear_residual(x, f(qw), f(s), f(z), None, r, G, "hip")
        assert out.shape == (2, 3, 64) and out.dtype == torch.float16
        out = torch.ops.tokenforge.w4a16_linear_silu_mul(x, f(qw), f(s), f(z), None, G, "hip")
        assert out.shape == (2, 3, 32) and out.dtype == torch.float16
        x8 = f(torch.zeros((2, 3, 256), dtype=torch.float8_e4m3fn))
        sc = f(torch.ones((2, 3, 1), dtype=torch.float32))
        out = torch.ops.tokenforge.w4a8_linear(x8, sc, f(qw), f(s), f(z), None, G, "hip")
        assert out.shape == (2, 3, 64) and out.dtype == torch.float16
        out = torch.ops.tokenforge.w4a8_linear(x8, sc, f(qw), f(s), f(z), None, G, "hip", "silu_mul")
        assert out.shape == (2, 3, 32)
        gamma = f(torch.ones(256, dtype=torch.float16))
        q, qs, a = torch.ops.tokenforge.rmsnorm_fp8_quant_dequant(x, gamma, 1e-6, None)
        assert q.shape == (2, 3, 256) and q.dtype == torch.float8_e4m3fn
        assert qs.shape == (2, 3, 1) and qs.dtype == torch.float32
        assert a.shape == (2, 3, 256) and a.dtype == torch.float16
        q, qs, a = torch.ops.tokenforge.rmsnorm_fp8_quant_dequant(x, gamma, 1e-6, f(torch.ones(1)))
        assert qs.shape == (1,) and a.shape == (2, 3, 256)


def test_rejects_marlin_at_op_level() -> None:
    qw, s, z = _layer(torch.device("cpu"))
    with pytest.raises(ValueError, match="op level"):
        torch.ops.tokenforge.w4a16_linear(cases.activations(1, 256, 0), qw, s, z, None, G, "marlin")


def test_schema_matches_reference() -> None:
    schema = str(torch.ops.tokenforge.w4a16_linear.default._schema)
    assert schema == (
        "tokenforge::w4a16_linear(Tensor x, Tensor qweight_t, Tensor scales, Tensor qzeros, "
        "Tensor? bias, SymInt group_size, str backend) -> Tensor"
    )
    assert str(torch.ops.tokenforge.w4a16_dequant.default._schema) == (
        "tokenforge::w4a16_dequant(Tensor qweight_t, Tensor scales, Tensor qzeros, SymInt group_size) -> Tensor"
    )
    assert str(torch.ops.tokenforge.rmsnorm_fp8_quant.default._schema) == (
        "tokenforge::rmsnorm_fp8_quant(Tensor x, Tensor weight, float eps, Tensor? scale) -> (Tensor, Tensor)"
    )


@pytest.mark.gpu
@pytest.mark.parametrize("with_bias", [False, True])
def test_opcheck_w4a16_linear(with_bias: bool, device: torch.device) -> None:
    qw, s, z = _layer(device)
    x = cases.activations(3, 256, 0).to(device)
    b = cases.bias(64, 0).to(device) if with_bias else None
    opcheck(torch.ops.tokenforge.w4a16_linear.default, (x, qw, s, z, b, G, "hip"), test_utils=OPCHECK_TESTS)


@pytest.mark.gpu
def test_opcheck_dequant_and_rmsnorm(device: torch.device) -> None:
    qw, s, z = _layer(device)
    opcheck(torch.ops.tokenforge.w4a16_dequant.default, (qw, s, z, G), test_utils=OPCHECK_TESTS)
    x = cases.activations(4, 256, 1).to(device)
    w = torch.ones(256, dtype=torch.float16, device=device)
    opcheck(
        torch.ops.tokenforge.rmsnorm_fp8_quant.default,
        (x, w, 1e-6, None),
        test_utils=("test_schema", "test_faketensor"),
    )


@pytest.mark.gpu
def test_opcheck_added_ops(device: torch.device) -> None:
    qw, s, z = _layer(device)
    x = cases.activations(3, 256, 0).to(device)
    r = cases.activations(3, 64, 1).to(device)
    b = cases.bias(64, 0).to(device)
    ops = torch.ops.tokenforge
    opcheck(ops.w4a16_linear_residual.default, (x, qw, s, z, b, r, G, "hip"), test_utils=OPCHECK_TESTS)
    opcheck(ops.w4a16_linear_silu_mul.default, (x, qw, s, z, None, G, "hip"), test_utils=OPCHECK_TESTS)
    q8, sc = ops.rmsnorm_fp8_quant(x, torch.ones(256, dtype=torch.float16, device=device), 1e-6, None)
    # opcheck's schema test does arithmetic on the inputs, which torch has no kernel for in
    # float8_e4m3fn; the fake-tensor and dynamic-shape AOT checks run.
    w4a8_tests = ("test_faketensor", "test_aot_dispatch_dynamic")
    opcheck(ops.w4a8_linear.default, (q8, sc, qw, s, z, b, G, "hip"), test_utils=w4a8_tests)
    opcheck(ops.w4a8_linear.default, (q8, sc, qw, s, z, None, G, "hip", "residual", r), test_utils=w4a8_tests)
    gamma = torch.ones(256, dtype=torch.float16, device=device)
    opcheck(ops.rmsnorm_fp8_quant_dequant.default, (x, gamma, 1e-6, None), test_utils=w4a8_tests)
    opcheck(ops.rmsnorm_fp8_quant_dequant.default, (x, gamma, 1e-6, torch.full((1,), 0.01, device=device)),
            test_utils=w4a8_tests)


class _QLinear(torch.nn.Module):
    def __init__(self, device: torch.device) -> None:
        super().__init__()
        qw, s, z = _layer(device)
        self.register_buffer("qw", qw)
        self.register_buffer("s", s)
        self.register_buffer("z", z)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        h = torch.ops.tokenforge.w4a16_linear(x, self.qw, self.s, self.z, None, G, "hip")
        return torch.relu(h) * 2


@pytest.mark.gpu
def test_torch_compile_fullgraph_no_graph_breaks(device: torch.device) -> None:
    mod = _QLinear(device)
    x = cases.activations(5, 256, 2).to(device)
    eager = mod(x)
    compiled = torch.compile(mod, backend="aot_eager", fullgraph=True, dynamic=True)
    assert torch.equal(compiled(x), eager)
    # A new M must reuse the dynamic graph and still dispatch by its own bucket.
    KERNEL_CALLS.reset()
    x2 = cases.activations(17, 256, 3).to(device)
    assert torch.equal(compiled(x2), mod(x2))
    # Bucket 32 is served by either family (the tuned config decides; untuned it is the GEMM).
    calls = [KERNEL_CALLS.value(kernel=k, bucket="32") for k in ("hip_gemv", "hip_gemm")]
    assert sum(calls) == 2


class _FusedMlp(torch.nn.Module):
    """RMSNorm + FP8 -> W4A8 gate_up with SiLU*mul -> W4A16 down with the residual add."""

    def __init__(self, device: torch.device) -> None:
        super().__init__()
        gq, gs, gz = _layer(device, 512, 256)  # gate and up halves of 256 each
        dq, ds, dz = _layer(device, 256, 256)
        for name, t in (("gq", gq), ("gs", gs), ("gz", gz), ("dq", dq), ("ds", ds), ("dz", dz)):
            self.register_buffer(name, t)
        self.register_buffer("gamma", torch.ones(256, dtype=torch.float16, device=device))

    def forward(self, h: torch.Tensor) -> torch.Tensor:
        ops = torch.ops.tokenforge
        q8, sc = ops.rmsnorm_fp8_quant(h, self.gamma, 1e-6, None)
        act = ops.w4a8_linear(q8, sc, self.gq, self.gs, self.gz, None, G, "hip", "silu_mul")
        return ops.w4a16_linear_residual(act, self.dq, self.ds, self.dz, None, h, G, "hip")


@pytest.mark.gpu
def test_torch_compile_fullgraph_added_ops(device: torch.device) -> None:
    mod = _FusedMlp(device)
    h = cases.activations(5, 256, 4).to(device)
    compiled = torch.compile(mod, backend="aot_eager", fullgraph=True, dynamic=True)
    assert torch.equal(compiled(h), mod(h))
    h2 = cases.activations(9, 256, 5).to(device)
    assert torch.equal(compiled(h2), mod(h2))
