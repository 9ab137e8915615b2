"""T0: AWQ packing, the TokenForge layout and dequantization.

CPU tests pin the oracle (oracle/pack.py) the way the reference's tests/unit/test_pack.py
pins its own code: an independent scalar packing loop written from AutoAWQ's published
``WQLinear_GEMM`` packing order, the sign-bit known answer, round trips, element
consistency of the two layouts, group-boundary and zero-point-extreme known answers and
the quantizer's error bound. GPU tests check the product's HIP kernels bit-exact against
the pinned oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import pack as P
from tests.numerics import cases

G = 128


def _scalar_autoawq_pack(intweight: np.ndarray) -> np.ndarray:
    """AutoAWQ's GEMM packing written out element by element: for every group of 8 output
    columns, nibble i of the word holds column ``order[i]``, order = [0, 2, 4, 6, 1, 3, 5, 7]."""
    k, n = intweight.shape
    order = [0, 2, 4, 6, 1, 3, 5, 7]
    out = np.zeros((k, n // 8), dtype=np.int64)
    for row in range(k):
        for col in range(n // 8):
            word = 0
            for i in range(8):
                word |= int(intweight[row, col * 8 + order[i]]) << (4 * i)
            out[row, col] = word
    return out.astype(np.uint32).view(np.int32)


def test_orders_are_inverse() -> None:
    assert [P.AWQ_ORDER[P.AWQ_REVERSE_ORDER[j]] for j in range(8)] == list(range(8))
    assert list(P.AWQ_REVERSE_ORDER) == [(j % 2) * 4 + j // 2 for j in range(8)]


@settings(max_examples=60, deadline=None)
@given(rows=st.integers(1, 9), words=st.integers(1, 6), seed=st.integers(0, 2**31 - 1))
def test_pack_roundtrip(rows: int, words: int, seed: int) -> None:
    rng = np.random.default_rng(seed)
    values = rng.integers(0, 16, (rows, words * 8), dtype=np.int32)
    values[0, 0], values[-1, -1] = 0, 15
    packed = P.pack_int4(values)
    assert packed.dtype == np.int32
    assert packed.shape == (rows, words)
    assert np.array_equal(P.unpack_int4(packed), values)


@settings(max_examples=25, deadline=None)
@given(k=st.integers(1, 6), n_words=st.integers(1, 5), seed=st.integers(0, 2**31 - 1))
def test_awq_pack_matches_scalar_autoawq_loop(k: int, n_words: int, seed: int) -> None:
    rng = np.random.default_rng(seed)
    intweight = rng.integers(0, 16, (k, n_words * 8), dtype=np.int32)
    zeros = rng.integers(0, 16, (1, n_words * 8), dtype=np.int32)
    qweight, _ = P.awq_pack(intweight, zeros)
    assert np.array_equal(qweight, _scalar_autoawq_pack(intweight))
    assert np.array_equal(P.awq_unpack(qweight), intweight)


def test_high_nibble_sign_bit() -> None:
    """15 in nibble 7 sets bit 31; the pattern must survive int32 wrap-around."""
    values = np.zeros((1, 8), dtype=np.int32)
    values[0, P.AWQ_ORDER[7]] = 15
    packed = P.pack_int4(values)
    assert int(packed[0, 0]) == -(2**28)  # 0xF0000000 as int32
    assert np.array_equal(P.unpack_int4(packed), values)


def test_pack_rejects_out_of_range() -> None:
    with pytest.raises(ValueError, match=r"\[0, 15\]"):
        P.pack_int4(np.full((1, 8), 16, dtype=np.int32))
    with pytest.raises(ValueError, match="multiple of 8"):
        P.pack_int4(np.zeros((1, 7), dtype=np.int32))


@settings(max_examples=20, deadline=None)
@given(k_groups=st.integers(1, 3), n_words=st.integers(1, 4), seed=st.integers(0, 2**31 - 1))
def test_repack_is_invertible(k_groups: int, n_words: int, seed: int) -> None:
    rng = np.random.default_rng(seed)
    k, n = k_groups * G, n_words * 8
    qweight = rng.integers(-(2**31), 2**31 - 1, (k, n // 8), dtype=np.int64).astype(np.int32)
    qweight_t = P.repack_awq_to_tf(qweight)
    assert qweight_t.shape == (n, k // 8)
    assert np.array_equal(P.repack_tf_to_awq(qweight_t), qweight)
    # Element (k, n) of the logical matrix is the same in both layouts.
    assert np.array_equal(P.unpack_int4(qweight_t).T, P.awq_unpack(qweight))


def test_repack_brute_force_single_nibbles() -> None:
    """Each single set nibble of a 16x16 matrix lands at its transposed position."""
    for kk in range(16):
        for nn in range(16):
            logical = np.zeros((16, 16), dtype=np.int32)
            logical[kk, nn] = 9
            qweight = P.pack_int4(logical)
            qt = P.repack_awq_to_tf(qweight)
            word = int(qt[nn, kk // 8]) & 0xFFFFFFFF
            assert word == 9 << (4 * P.AWQ_REVERSE_ORDER[kk % 8])
            assert np.count_nonzero(qt) == 1


def _random_awq(n: int, k: int, seed: int, group: int = G) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    rng = np.random.default_rng(seed)
    intweight = rng.integers(0, 16, (k, n), dtype=np.int32)
    zeros = rng.integers(0, 16, (k // group, n), dtype=np.int32)
    zeros[0, 0], zeros[-1, -1] = 0, 15
    scales = (rng.random((k // group, n), dtype=np.float32) * 0.01 + 1e-3).astype(np.float16)
    qweight, qzeros = P.awq_pack(intweight, zeros)
    return qweight, qzeros, scales


def test_pack_awq_roundtrip_and_dequant_agree() -> None:
    qweight, qzeros, scales = _random_awq(n=64, k=3 * G, seed=7)
    w = P.pack_awq(qweight, qzeros, scales, G)
    assert (w.n, w.k) == (64, 3 * G)
    back = P.unpack_to_awq(w)
    assert np.array_equal(back[0], qweight)
    assert np.array_equal(back[1], qzeros)
    assert np.array_equal(back[2], scales)
    assert np.array_equal(P.dequantize_tf(w), P.awq_dequantize(qweight, qzeros, scales, G).T)


def test_dequant_at_group_boundaries() -> None:
    qweight, qzeros, scales = _random_awq(n=16, k=2 * G, seed=3)
    q = P.awq_unpack(qweight)
    z = P.awq_unpack(qzeros)
    deq = P.awq_dequantize(qweight, qzeros, scales, G)
    for kk in (0, G - 1, G, 2 * G - 1):
        g = kk // G
        for nn in (0, 7, 8, 15):
            expected = np.float16(float(q[kk, nn] - z[g, nn])) * scales[g, nn]
            assert deq[kk, nn] == expected, (kk, nn)


def test_zero_points_at_extremes() -> None:
    k, n = G, 8
    intweight = np.array([[0, 15, 0, 15, 7, 8, 1, 14]] * k, dtype=np.int32)
    for zp in (0, 15):
        zeros = np.full((1, n), zp, dtype=np.int32)
        qweight, qzeros = P.awq_pack(intweight, zeros)
        scales = np.ones((1, n), dtype=np.float16)
        deq = P.awq_dequantize(qweight, qzeros, scales, G)
        assert np.array_equal(deq[0], (intweight[0] - zp).astype(np.float16))


def test_awq_quantize_error_bound() -> None:
    gen = torch.Generator().manual_seed(0)
    weight = (torch.randn((32, 2 * G), generator=gen) * 0.05).numpy()
    qweight, qzeros, scales = P.awq_quantize(weight, G)
    P.validate_awq(qweight, qzeros, scales, G)
    deq = P.awq_dequantize(qweight, qzeros, scales, G).T.astype(np.float32)  # [N, K]
    step = np.repeat(scales.astype(np.float32), G, axis=0).T
    assert bool((np.abs(deq - weight) <= 0.5 * step + 1e-3 * step + 1e-6).all())


def test_awq_quantize_scalar_rederivation() -> None:
    """Scale, zero and codes of a few groups recomputed with scalar fp32 arithmetic."""
    gen = torch.Generator().manual_seed(3)
    weight = (torch.randn((8, 2 * G), generator=gen) * 0.02).numpy()
    qweight, qzeros, scales = P.awq_quantize(weight, G)
    q = P.awq_unpack(qweight)
    z = P.awq_unpack(qzeros)
    for row in (0, 5):
        for g in (0, 1):
            grp = weight[row, g * G:(g + 1) * G].astype(np.float32)
            s32 = np.float32(np.float16(max(np.float32(grp.max() - grp.min()), np.float32(1e-5)) / np.float32(15)))
            zero = min(max(-round(float(np.float32(grp.min() / s32))), 0), 15)
            assert float(scales[g, row]) == float(s32)
            assert int(z[g, row]) == zero
            for kk in (0, 17, G - 1):
                code = min(max(round(float(np.float32(grp[kk] / s32))) + zero, 0), 15)
                assert int(q[g * G + kk, row]) == code


@pytest.mark.parametrize(
    ("mutate", "match"),
    [
        (lambda q, z, s: (q.astype(np.float32), z, s), "int32"),
        (lambda q, z, s: (q, z, s.astype(np.float32)), "fp16"),
        (lambda q, z, s: (q, z[:1], s), "qzeros shape"),
        (lambda q, z, s: (q, z, s[:, :8]), "scales shape"),
    ],
)
def test_validate_awq_rejects(mutate, match) -> None:  # type: ignore[no-untyped-def]
    qweight, qzeros, scales = _random_awq(n=16, k=2 * G, seed=1)
    with pytest.raises(ValueError, match=match):
        P.validate_awq(*mutate(qweight, qzeros, scales), G)


def test_validate_awq_rejects_group_and_k() -> None:
    qweight, qzeros, scales = _random_awq(n=16, k=2 * G, seed=1)
    with pytest.raises(ValueError, match="group_size"):
        P.validate_awq(qweight, qzeros, scales, 256)
    with pytest.raises(ValueError, match="multiple of group_size"):
        P.validate_awq(qweight[:-8], qzeros, scales, G)


# ------------------------------------------------------------------ gfx950 tile layout (oracle)

TILE_SHAPES = [(16, 128, 128), (8, 32, 32), (24, 96, 32), (40, 192, 64), (200, 256, 128), (48, 160, 32), (64, 384, 64)]


@pytest.mark.parametrize(("n", "k", "group"), TILE_SHAPES)
def test_tile_layout_formula_matches_its_storage_order(n: int, k: int, group: int) -> None:
    """The closed-form positions equal the storage order that defines the layout (tile by
    tile, K step by step, chunk column by column, row by row), for every chunk, scale and zero
    word, so each map is a bijection."""
    q_total, p_total = k // 32, k // group
    for i, (row, q) in enumerate(P.tile_order_chunks(n, q_total)):
        assert P.tile_chunk_index(np.array(row), np.array(q), n, q_total) == i
    assert len(P.tile_order_chunks(n, q_total)) == n * q_total
    for i, (grp, row) in enumerate(P.tile_order_scales(n, p_total)):
        assert P.tile_scale_index(np.array(grp), np.array(row), n, p_total) == i
    for i, (grp, word) in enumerate(P.tile_order_zeros(n, p_total)):
        assert P.tile_zero_index(np.array(grp), np.array(word), n, p_total) == i
    assert len(P.tile_order_zeros(n, p_total)) == p_total * n // 8


@pytest.mark.parametrize(("n", "k", "group"), TILE_SHAPES)
def test_tile_layout_round_trip_and_content(n: int, k: int, group: int) -> None:
    rng = np.random.default_rng(n * 31 + k)
    qw = rng.integers(-(2**31), 2**31 - 1, (n, k // 8), dtype=np.int64).astype(np.int32)
    sc = rng.random((k // group, n)).astype(np.float16)
    qz = rng.integers(-(2**31), 2**31 - 1, (k // group, n // 8), dtype=np.int64).astype(np.int32)
    tiled = P.tile_pack(qw, sc, qz, group)
    assert [t.shape for t in tiled] == [qw.shape, sc.shape, qz.shape]
    back = P.tile_unpack(*tiled, group)
    assert all(np.array_equal(a, b) for a, b in zip(back, (qw, sc, qz)))
    # Chunk content is untouched: the multiset of 16-byte chunks is the same.
    rows = lambda a: sorted(map(bytes, a.reshape(-1, 4)))  # noqa: E731
    assert rows(tiled[0]) == rows(qw)


def test_tile_layout_step_blocks_are_the_mfma_operand() -> None:
    """A full tile's 128-wide K step is one contiguous 1 KB block whose 16-byte slot l holds
    row l % 16, K offsets 128 j + 32 (l // 16) .. + 31: the B operand of lane l."""
    n, k = 48, 512
    rng = np.random.default_rng(1)
    vals = rng.integers(0, 16, (n, k), dtype=np.int32)
    qw = P.pack_int4(vals)  # TokenForge layout [N, K/8]
    tiled, _, _ = P.tile_pack(qw, np.zeros((k // 128, n), np.float16), np.zeros((k // 128, n // 8), np.int32), 128)
    flat = tiled.reshape(-1, 4)  # 16-byte slots
    q_total = k // 32
    for t in range(n // 16):
        for j in range(k // 128):
            block = flat[16 * t * q_total + 64 * j: 16 * t * q_total + 64 * (j + 1)]
            for lane in range(64):
                row, g = 16 * t + lane % 16, lane // 16
                want = vals[row, 128 * j + 32 * g: 128 * j + 32 * g + 32]
                assert np.array_equal(P.unpack_int4(block[lane]), want)


def test_tile_layout_pack_awq_tiles_dequantizes_like_the_reference() -> None:
    qweight, qzeros, scales = _random_awq(n=40, k=256, seed=3, group=64)
    tiled = P.pack_awq_tiles(qweight, qzeros, scales, 64)
    back = P.tile_unpack(tiled.qweight_t, tiled.scales, tiled.qzeros, 64)
    ref = P.pack_awq(qweight, qzeros, scales, 64)
    assert np.array_equal(back[0], ref.qweight_t)
    assert np.array_equal(back[2], ref.qzeros)


# ------------------------------------------------------------------ product on the GPU


def _t(a: np.ndarray, device: torch.device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


@pytest.mark.gpu
@pytest.mark.parametrize(("k", "n"), [(8, 8), (128, 64), (264, 200), (384, 1000), (2048, 520), (4096, 256)])
def test_gpu_repack_bit_exact(k: int, n: int, device: torch.device) -> None:
    from tokenforge.kernels import pack as tp

    rng = np.random.default_rng(k * 7 + n)
    qweight = rng.integers(-(2**31), 2**31 - 1, (k, n // 8), dtype=np.int64).astype(np.int32)
    qt = tp.repack_awq_to_tf(_t(qweight, device))
    assert np.array_equal(qt.cpu().numpy(), P.repack_awq_to_tf(qweight))
    back = tp.repack_tf_to_awq(qt)
    assert np.array_equal(back.cpu().numpy(), qweight)


@pytest.mark.gpu
def test_gpu_pack_unpack_and_range_check(device: torch.device) -> None:
    from tokenforge.kernels import pack as tp

    rng = np.random.default_rng(0)
    values = rng.integers(0, 16, (37, 96), dtype=np.int32)
    packed = tp.pack_int4(_t(values, device))
    assert np.array_equal(packed.cpu().numpy(), P.pack_int4(values))
    assert np.array_equal(tp.unpack_int4(packed).cpu().numpy(), values)
    bad = values.copy()
    bad[3, 5] = 16
    with pytest.raises(ValueError, match=r"\[0, 15\]"):
        tp.pack_int4(_t(bad, device))
    with pytest.raises(ValueError, match="multiple of 8"):
        tp.pack_int4(_t(values[:, :7], device))
    with pytest.raises(TypeError, match="int32"):
        tp.unpack_int4(_t(values.astype(np.int64), device))


@pytest.mark.gpu
@pytest.mark.parametrize(("n", "k", "group"), [(200, 3 * G, G), (64, 96, 32), (40, 192, 64), (256, 4 * G, G)])
def test_gpu_pack_awq_tile_layout_and_dequant_bit_exact(n: int, k: int, group: int, device: torch.device) -> None:
    """pack_awq emits the gfx950 tile layout bit for bit as the oracle restates it (ragged N,
    K not a multiple of 128), unpack_to_awq inverts it, and the dequant reading the tile layout
    equals the reference's dequantize_tf on the TokenForge layout."""
    from tokenforge.kernels import pack as tp

    qweight, qzeros, scales = _random_awq(n=n, k=k, seed=11 + n, group=group)
    w = tp.pack_awq(_t(qweight, device), _t(qzeros, device), _t(scales, device), group)
    ow = P.pack_awq_tiles(qweight, qzeros, scales, group)
    assert np.array_equal(w.qweight_t.cpu().numpy(), ow.qweight_t)
    assert np.array_equal(w.scales.cpu().numpy().view(np.uint16), ow.scales.view(np.uint16))
    assert np.array_equal(w.qzeros.cpu().numpy(), ow.qzeros)
    assert (w.n, w.k) == (n, k)
    ref = P.dequantize_tf(P.pack_awq(qweight, qzeros, scales, group))
    assert np.array_equal(tp.dequantize_tf(w).cpu().numpy().view(np.uint16), ref.view(np.uint16))
    assert np.array_equal(
        tp.awq_dequantize(_t(qweight, device), _t(qzeros, device), _t(scales, device), group).cpu().numpy(),
        P.awq_dequantize(qweight, qzeros, scales, group),
    )
    back = tp.unpack_to_awq(w)
    assert np.array_equal(back[0].cpu().numpy(), qweight)
    assert np.array_equal(back[1].cpu().numpy(), qzeros)
    assert np.array_equal(back[2].cpu().numpy().view(np.uint16), scales.view(np.uint16))
    with pytest.raises(ValueError, match="qzeros shape"):
        tp.pack_awq(_t(qweight, device), _t(qzeros[:1], device), _t(scales, device), group)


@pytest.mark.gpu
def test_gpu_load_time_functions_accept_host_tensors(device: torch.device) -> None:
    """Like the reference's, the load-time functions take host tensors: the kernel runs on the
    GPU and the result comes back on the host, bit-exact."""
    from tokenforge.kernels import pack as tp

    qweight, qzeros, scales = _random_awq(n=64, k=2 * G, seed=5)
    qt = tp.repack_awq_to_tf(torch.from_numpy(qweight))
    assert qt.device.type == "cpu" and np.array_equal(qt.numpy(), P.repack_awq_to_tf(qweight))
    w = tp.pack_awq(torch.from_numpy(qweight), torch.from_numpy(qzeros), torch.from_numpy(scales), G)
    assert w.qweight_t.device.type == "cpu"
    assert np.array_equal(w.qweight_t.numpy(), P.pack_awq_tiles(qweight, qzeros, scales, G).qweight_t)
    assert np.array_equal(tp.dequantize_tf(w).numpy(), P.dequantize_tf(P.pack_awq(qweight, qzeros, scales, G)))


@pytest.mark.gpu
@pytest.mark.parametrize(("n", "k", "group"), [(64, 256, 128), (200, 384, 64), (48, 96, 32), (1024, 1024, 128)])
def test_gpu_awq_quantize_bit_exact(n: int, k: int, group: int, device: torch.device) -> None:
    """awq_quantize (pack.py:83-107) on the GPU equals the oracle's fp32 restatement bit for bit,
    on the device and from host tensors."""
    from tokenforge.kernels import pack as tp

    gen = torch.Generator().manual_seed(n + k + group)
    weight = torch.randn((n, k), generator=gen) * 0.02
    weight[0, :group] = 0.0  # a constant group: the 1e-5 clamp of the range
    want = P.awq_quantize(weight.numpy(), group)
    for got in (tp.awq_quantize(weight.to(device), group), tp.awq_quantize(weight, group)):
        assert np.array_equal(got[0].cpu().numpy(), want[0])
        assert np.array_equal(got[1].cpu().numpy(), want[1])
        assert np.array_equal(got[2].cpu().numpy().view(np.uint16), want[2].view(np.uint16))
    with pytest.raises(ValueError, match="multiple of group_size"):
        tp.awq_quantize(weight[:, :-8].to(device), group)


@pytest.mark.gpu
@pytest.mark.parametrize(
    ("layer", "n", "k"),
    [("qkv", 4608, 3584), ("o", 3584, 3584), ("gate_up", 37888, 3584), ("down", 3584, 18944)],
)
def test_gpu_repack_qwen7b_full_size(layer: str, n: int, k: int, device: torch.device) -> None:
    """AWQ repack of every Qwen2.5-7B decoder linear, bit-exact."""
    from tokenforge.kernels import pack as tp

    qweight, qzeros, scales = cases.baseline_layer(n, k, seed=0)
    qt = tp.repack_awq_to_tf(_t(qweight, device)).cpu().numpy()
    assert np.array_equal(qt, P.repack_awq_to_tf(qweight)), layer
    # ... and pack_awq's tile layout, bit-exact, with an exact round trip back to AWQ.
    w = tp.pack_awq(_t(qweight, device), _t(qzeros, device), _t(scales, device), G)
    want = P.tile_pack(qt, scales, qzeros, G)
    assert np.array_equal(w.qweight_t.cpu().numpy(), want[0]), layer
    assert np.array_equal(w.scales.cpu().numpy().view(np.uint16), want[1].view(np.uint16)), layer
    assert np.array_equal(w.qzeros.cpu().numpy(), want[2]), layer
    back = tp.unpack_to_awq(w)
    for got, ref in zip(back, (qweight, qzeros, scales)):
        assert np.array_equal(got.cpu().numpy().view(np.int16), ref.view(np.int16)), layer
