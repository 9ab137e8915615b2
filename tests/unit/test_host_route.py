"""The torch route for host tensors (tokenforge/kernels/host.py) against the oracle, on CPU.

The reference runs host tensors through torch (dispatch.py:90-91 -> ops.py:79-81,
reference.py:24-56; pack.py's torch layout functions). Here the ops and, with no GPU visible,
the load-time layout functions do the same through ``tokenforge.kernels.host``:

* the int4 packing, the AWQ <-> TokenForge repack, the gfx950 tile layout, the AWQ quantizer and
  the dequantization are bit-exact against the oracle (oracle/pack.py);
* the linear is held to the fp64 oracle (oracle/reference.py::w4a16_reference) within the
  error of an fp32 dot product of length K plus one fp16 rounding; its epilogues equal their
  unfused torch expressions bit for bit;
* the norm's codes are within one e4m3 code of the oracle's on fewer than 0.1% of elements
  (the allowance between the reference's torch order and an exact sum), its scales within one
  fp32 ulp;
* the reference's CPU op tests run: opcheck and torch.compile(fullgraph) on host tensors.

These tests run in the CPU container; with a GPU visible the load-time functions would send
host tensors to it instead, so the layout checks call the torch route directly as well.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch.library import opcheck

import tokenforge.kernels.ops  # noqa: F401
from oracle import pack as opack
from oracle import reference as oref
from tests.numerics import cases
from tokenforge.kernels import host
from tokenforge.kernels import pack as tpack
from tokenforge.kernels.metrics import KERNEL_CALLS

G = cases.GROUP_SIZE
CPU = torch.device("cpu")


def _t(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a))


def _layer(n: int, k: int, seed: int, g: int = G) -> tuple[opack.W4A16Weights, tpack.W4A16Weights]:
    ow = cases.layer_weights(n, k, seed, g)
    return ow, cases.on_device(ow, CPU)


def test_nibble_order_matches_the_package_constants() -> None:
    shifts = host._offset_shifts(CPU).tolist()
    assert shifts == [4 * tpack.AWQ_REVERSE_ORDER[j] for j in range(8)]
    assert [shifts.index(4 * i) for i in range(8)] == list(tpack.AWQ_ORDER)


@pytest.mark.parametrize("shape", [(3, 8), (5, 64), (2, 3, 16)])
def test_pack_unpack_int4_bit_exact(shape: tuple[int, ...]) -> None:
    gen = torch.Generator().manual_seed(sum(shape))
    v = torch.randint(0, 16, shape, generator=gen, dtype=torch.int32)
    v.view(-1)[:8] = 15  # a word with its top nibble set: a negative int32
    words = host.pack_int4(v)
    assert np.array_equal(words.numpy(), opack.pack_int4(v.numpy()))
    assert torch.equal(host.unpack_int4(words), v)
    assert torch.equal(tpack.pack_int4(v), words)  # the package function (torch route here)
    assert torch.equal(tpack.unpack_int4(words), v)


def test_pack_int4_rejects_what_the_reference_rejects() -> None:
    with pytest.raises(ValueError, match=r"\[0, 15\]"):
        host.pack_int4(torch.full((1, 8), 16, dtype=torch.int32))
    with pytest.raises(ValueError, match="multiple of 8"):
        host.pack_int4(torch.zeros((1, 12), dtype=torch.int32))
    with pytest.raises(TypeError, match="int32"):
        host.unpack_int4(torch.zeros((1, 2), dtype=torch.int64))


@pytest.mark.parametrize(("n", "k"), [(64, 256), (40, 128), (24, 384)])
def test_repack_and_tile_layout_bit_exact(n: int, k: int) -> None:
    """AWQ -> TokenForge -> tile layout and back, on N = 16t and 16t + 8 (a half last tile) and
    K with a last 128-wide step that is shorter (K = 384 = 3·128; 40 rows: tiles of 16, 16, 8)."""
    gen = torch.Generator().manual_seed(n + k)
    weight = (torch.randn((n, k), generator=gen) * 0.02).numpy()
    qweight, qzeros, scales = opack.awq_quantize(weight, G)
    tf = host.transpose_packed(_t(qweight))
    assert np.array_equal(tf.numpy(), opack.repack_awq_to_tf(qweight))
    assert np.array_equal(host.transpose_packed(tf).numpy(), qweight)
    tiled = host.tile_pack(tf, _t(scales), _t(qzeros), G)
    expect = opack.tile_pack(opack.repack_awq_to_tf(qweight), scales, qzeros, G)
    for got, want in zip(tiled, expect):
        assert np.array_equal(got.numpy(), want)
    for got, want in zip(host.tile_unpack(*tiled, G), (tf, _t(scales), _t(qzeros))):
        assert torch.equal(got, want)
    w = tpack.pack_awq(_t(qweight), _t(qzeros), _t(scales), G)  # the package entry (torch route)
    assert torch.equal(w.qweight_t, tiled[0]) and torch.equal(w.scales, tiled[1]) and torch.equal(w.qzeros, tiled[2])
    back = tpack.unpack_to_awq(w)
    assert np.array_equal(back[0].numpy(), qweight) and np.array_equal(back[1].numpy(), qzeros)


@pytest.mark.parametrize("g", [32, 64, 128])
def test_awq_quantize_and_dequantize_bit_exact(g: int) -> None:
    gen = torch.Generator().manual_seed(g)
    weight = torch.randn((48, 512), generator=gen) * 0.05
    weight[3, :g] = 0.0  # a constant group: the 1e-5 floor of the scale
    got = host.awq_quantize(weight, g)
    want = opack.awq_quantize(weight.numpy(), g)
    for a, b in zip(got, want):
        assert np.array_equal(a.numpy(), b)
    ow = opack.pack_awq(*want, g)
    w = cases.on_device(ow, CPU)
    deq = host.dequantize(w.qweight_t, w.scales, w.qzeros, g)
    assert np.array_equal(deq.numpy().view(np.uint16), opack.dequantize_tf(ow).view(np.uint16))
    op = torch.ops.tokenforge.w4a16_dequant(w.qweight_t, w.scales, w.qzeros, g)
    assert torch.equal(op.view(torch.int16), deq.view(torch.int16))


def _linear_bound(x: torch.Tensor, ow: opack.W4A16Weights, ref: np.ndarray) -> np.ndarray:
    """|fp16(fp32 dot) - exact| <= half an fp16 ulp of the result (2^-11 relative, the
    subnormal floor aside) + the fp32 summation error of a length-K dot product,
    K·2^-24·sum|x||w| (doubled for slack)."""
    k = x.shape[1]
    w = np.abs(opack.dequantize_tf(ow).astype(np.float64))
    mag = np.abs(x.numpy().astype(np.float64)) @ w.T
    return 2.0**-11 * np.abs(ref) + 2.0**-24 + 2 * k * 2.0**-24 * mag


@pytest.mark.parametrize(("m", "n", "k"), [(1, 64, 256), (7, 128, 512), (33, 96, 1024)])
def test_w4a16_linear_on_host_tensors(m: int, n: int, k: int) -> None:
    ow, w = _layer(n, k, m)
    x = cases.activations(m, k, m)
    b = cases.bias(n, m)
    KERNEL_CALLS.reset()
    y = torch.ops.tokenforge.w4a16_linear(x, w.qweight_t, w.scales, w.qzeros, b, G, "hip")
    assert y.dtype == torch.float16 and y.device.type == "cpu" and y.shape == (m, n)
    bucket = tokenforge.kernels.dispatch.bucket_label(m)
    assert KERNEL_CALLS.value(kernel="torch_reference", bucket=bucket) == 1
    ref = oref.w4a16_reference(x.numpy(), ow, b.numpy())
    err = np.abs(y.numpy().astype(np.float64) - ref)
    assert bool((err <= _linear_bound(x, ow, ref)).all())
    # A 3-D x keeps its leading dims.
    y3 = torch.ops.tokenforge.w4a16_linear(x.reshape(1, m, k), w.qweight_t, w.scales, w.qzeros, b, G, "hip")
    assert torch.equal(y3.reshape(m, n), y)


def test_fused_linear_forms_equal_their_torch_expressions_on_host() -> None:
    m, n, k = 5, 128, 256
    _, w = _layer(n, k, 3)
    x = cases.activations(m, k, 3)
    r = cases.activations(m, n, 4)
    ops = torch.ops.tokenforge
    y = ops.w4a16_linear(x, w.qweight_t, w.scales, w.qzeros, None, G, "hip")
    res = ops.w4a16_linear_residual(x, w.qweight_t, w.scales, w.qzeros, None, r, G, "hip")
    assert torch.equal(res, r + y)
    act = ops.w4a16_linear_silu_mul(x, w.qweight_t, w.scales, w.qzeros, None, G, "hip")
    assert torch.equal(act, torch.nn.functional.silu(y[:, : n // 2]) * y[:, n // 2:])


def test_w4a8_and_norm_fused_linear_on_host() -> None:
    m, n, k = 4, 64, 256
    ow, w = _layer(n, k, 5)
    x = cases.activations(m, k, 6)
    gamma = (1 + 0.1 * cases.activations(1, k, 7)[0]).to(torch.float16)
    ops = torch.ops.tokenforge
    q8, sc, a = ops.rmsnorm_fp8_quant_dequant(x, gamma, 1e-6, None)
    q8b, scb = ops.rmsnorm_fp8_quant(x, gamma, 1e-6, None)
    assert torch.equal(q8.view(torch.uint8), q8b.view(torch.uint8)) and torch.equal(sc, scb)
    assert torch.equal(a, (q8.to(torch.float32) * sc).to(torch.float16))
    y8 = ops.w4a8_linear(q8, sc, w.qweight_t, w.scales, w.qzeros, None, G, "hip")
    ref = oref.w4a8_reference(q8.view(torch.uint8).numpy(), sc.numpy(), ow)
    err = np.abs(y8.numpy().astype(np.float64) - ref)
    xa = torch.from_numpy(oref.e4m3_decode(q8.view(torch.uint8).numpy()) * sc.numpy())
    assert bool((err <= _linear_bound(xa, ow, ref)).all())
    fused = ops.rmsnorm_fp8_w4a16_linear(x, gamma, 1e-6, w.qweight_t, w.scales, w.qzeros, None, G, "hip", "none")
    assert torch.equal(fused, ops.w4a16_linear(a, w.qweight_t, w.scales, w.qzeros, None, G, "hip"))


@pytest.mark.parametrize(("t", "h"), [(1, 896), (17, 3584), (4, 1000)])
def test_rmsnorm_fp8_quant_on_host_tensors(t: int, h: int) -> None:
    gen = torch.Generator().manual_seed(t * h)
    x = (torch.randn((t, h), generator=gen) * 2).to(torch.float16)
    w = (torch.rand((h,), generator=gen) + 0.5).to(torch.float16)
    q, s = torch.ops.tokenforge.rmsnorm_fp8_quant(x, w, 1e-6, None)
    assert q.dtype == torch.float8_e4m3fn and s.shape == (t, 1)
    q_ref, s_ref = oref.rmsnorm_fp8_reference(x.numpy(), w.numpy(), 1e-6)
    codes = q.view(torch.uint8).numpy().astype(np.int32)
    # Distance in codes between same-sign values (the low 7 bits are ordered by magnitude).
    dist = np.where((codes ^ q_ref.astype(np.int32)) & 0x80, 255, np.abs((codes & 0x7F) - (q_ref & 0x7F)))
    assert int(dist.max()) <= 1 and float((dist > 0).mean()) < 1e-3
    ulps = np.abs(s.numpy().view(np.int32) - s_ref.view(np.int32))
    assert int(ulps.max()) <= 1
    # Static scale: the codes of y / scale, the scale returned as given (a copy).
    st = torch.tensor([0.02], dtype=torch.float32)
    qs, ss = torch.ops.tokenforge.rmsnorm_fp8_quant(x, w, 1e-6, st)
    assert torch.equal(ss, st) and ss.data_ptr() != st.data_ptr()
    q_st, _ = oref.rmsnorm_fp8_reference(x.numpy(), w.numpy(), 1e-6, st.numpy())
    dist = np.abs(qs.view(torch.uint8).numpy().astype(np.int32) - q_st.astype(np.int32))
    assert float((dist > 0).mean()) < 1e-3


def test_host_calls_check_their_inputs_as_the_kernels_do() -> None:
    _, w = _layer(64, 256, 0)
    x = cases.activations(2, 256, 0)
    ops = torch.ops.tokenforge
    with pytest.raises(TypeError, match="fp16"):
        ops.w4a16_linear(x.float(), w.qweight_t, w.scales, w.qzeros, None, G, "hip")
    with pytest.raises(ValueError, match="bias shape"):
        ops.w4a16_linear(x, w.qweight_t, w.scales, w.qzeros, cases.bias(32, 0), G, "hip")
    with pytest.raises(ValueError, match="scales shape"):
        ops.w4a16_dequant(w.qweight_t, w.scales[:, :32], w.qzeros, G)
    with pytest.raises(ValueError, match="weight shape"):
        ops.rmsnorm_fp8_quant(x, torch.ones(128, dtype=torch.float16), 1e-6, None)
    with pytest.raises(ValueError, match="op level"):
        ops.w4a16_linear(x, w.qweight_t, w.scales, w.qzeros, None, G, "marlin")


OPCHECK_TESTS = ("test_schema", "test_faketensor", "test_aot_dispatch_dynamic")


def test_opcheck_on_host_tensors() -> None:
    """The reference's CPU-tier op checks (tests/unit/test_ops.py there) on host tensors."""
    _, w = _layer(64, 256, 0)
    qw, s, z = w.qweight_t, w.scales, w.qzeros
    x = cases.activations(3, 256, 0)
    ops = torch.ops.tokenforge
    for b in (None, cases.bias(64, 0)):
        opcheck(ops.w4a16_linear.default, (x, qw, s, z, b, G, "hip"), test_utils=OPCHECK_TESTS)
    opcheck(ops.w4a16_dequant.default, (qw, s, z, G), test_utils=OPCHECK_TESTS)
    opcheck(ops.rmsnorm_fp8_quant.default, (cases.activations(4, 256, 1), torch.ones(256, dtype=torch.float16),
                                            1e-6, None), test_utils=("test_schema", "test_faketensor"))
    r = cases.activations(3, 64, 1)
    opcheck(ops.w4a16_linear_residual.default, (x, qw, s, z, None, r, G, "hip"), test_utils=OPCHECK_TESTS)
    opcheck(ops.w4a16_linear_silu_mul.default, (x, qw, s, z, None, G, "hip"), test_utils=OPCHECK_TESTS)


class _QLinear(torch.nn.Module):
    def __init__(self) -> None:
        super().__init__()
        _, w = _layer(64, 256, 0)
        self.register_buffer("qw", w.qweight_t)
        self.register_buffer("s", w.scales)
        self.register_buffer("z", w.qzeros)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        h = torch.ops.tokenforge.w4a16_linear(x, self.qw, self.s, self.z, None, G, "hip")
        return torch.relu(h) * 2


def test_torch_compile_fullgraph_on_host_tensors() -> None:
    mod = _QLinear()
    x = cases.activations(5, 256, 2)
    compiled = torch.compile(mod, backend="aot_eager", fullgraph=True, dynamic=True)
    assert torch.equal(compiled(x), mod(x))
    KERNEL_CALLS.reset()
    x2 = cases.activations(17, 256, 3)
    assert torch.equal(compiled(x2), mod(x2))
    assert KERNEL_CALLS.value(kernel="torch_reference", bucket="32") == 2


@pytest.mark.gpu
def test_host_and_gpu_routes_agree(device: torch.device) -> None:
    """On a GPU box: the load-time functions send host tensors to the kernels, which return the
    torch route's bits; the ops' two routes agree within their error bounds; a call mixing host
    and GPU tensors raises."""
    n, k = 96, 512
    gen = torch.Generator().manual_seed(11)
    weight = torch.randn((n, k), generator=gen) * 0.02
    awq = tpack.awq_quantize(weight, G)  # host tensors in, the GPU kernel runs
    for a, b in zip(awq, host.awq_quantize(weight, G)):
        assert a.device.type == "cpu" and torch.equal(a, b)
    w_gpu_route = tpack.pack_awq(*awq[:2], awq[2], G)
    w_host = host.tile_pack(host.transpose_packed(awq[0]), awq[2], awq[1], G)
    for a, b in zip((w_gpu_route.qweight_t, w_gpu_route.scales, w_gpu_route.qzeros), w_host):
        assert torch.equal(a, b)
    ow = opack.pack_awq(*(a.numpy() for a in awq), G)
    x = cases.activations(6, k, 12)
    y_host = torch.ops.tokenforge.w4a16_linear(x, *w_host, None, G, "hip")
    y_gpu = torch.ops.tokenforge.w4a16_linear(x.to(device), *(t.to(device) for t in w_host), None, G, "hip")
    ref = oref.w4a16_reference(x.numpy(), ow)
    bound = _linear_bound(x, ow, ref)
    for y in (y_host, y_gpu.cpu()):
        assert bool((np.abs(y.numpy().astype(np.float64) - ref) <= bound).all())
    with pytest.raises(ValueError, match="one device"):
        torch.ops.tokenforge.w4a16_linear(x, *(t.to(device) for t in w_host), None, G, "hip")
    gamma = torch.ones(k, dtype=torch.float16)
    q_h, s_h = torch.ops.tokenforge.rmsnorm_fp8_quant(x, gamma, 1e-6, None)
    q_g, s_g = torch.ops.tokenforge.rmsnorm_fp8_quant(x.to(device), gamma.to(device), 1e-6, None)
    diff = q_h.view(torch.uint8).numpy().astype(np.int32) - q_g.cpu().view(torch.uint8).numpy().astype(np.int32)
    assert int(np.abs(diff).max()) <= 1 and float((diff != 0).mean()) < 1e-3
    assert int(np.abs(s_h.numpy().view(np.int32) - s_g.cpu().numpy().view(np.int32)).max()) <= 1
