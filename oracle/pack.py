"""Numpy restatement of the reference's AWQ packing and TokenForge layout (pack.py:1-194).

Test infrastructure only (see ``oracle/__init__.py``). All arrays are numpy; int4 words are
int32 two's-complement bit patterns, fp16 arrays are ``np.float16``.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

AWQ_ORDER: tuple[int, ...] = (0, 2, 4, 6, 1, 3, 5, 7)  # pack.py:32
AWQ_REVERSE_ORDER: tuple[int, ...] = (0, 4, 1, 5, 2, 6, 3, 7)  # pack.py:35
PACK_FACTOR = 8  # pack.py:38
SUPPORTED_GROUP_SIZES: tuple[int, ...] = (32, 64, 128)  # pack.py:39


def pack_int4(values: np.ndarray) -> np.ndarray:
    """pack.py:42-54: word = sum_i v[..., AWQ_ORDER[i]] << 4i, as an int32 bit pattern."""
    values = np.asarray(values)
    if values.shape[-1] % PACK_FACTOR != 0:
        raise ValueError(f"last dim {values.shape[-1]} is not a multiple of {PACK_FACTOR}")
    if values.size and (int(values.min()) < 0 or int(values.max()) > 15):
        raise ValueError("int4 values must lie in [0, 15]")
    *lead, n = values.shape
    v = values.astype(np.uint32).reshape(*lead, n // PACK_FACTOR, PACK_FACTOR)
    word = np.zeros(v.shape[:-1], dtype=np.uint32)
    for nibble, offset in enumerate(AWQ_ORDER):
        word |= v[..., offset] << np.uint32(4 * nibble)
    return word.view(np.int32)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """pack.py:57-67: value j = (word >> 4 * AWQ_REVERSE_ORDER[j]) & 0xF, int32."""
    packed = np.asarray(packed)
    if packed.dtype != np.int32:
        raise TypeError(f"packed tensor must be int32, got {packed.dtype}")
    shifts = np.array([4 * AWQ_REVERSE_ORDER[j] for j in range(PACK_FACTOR)], dtype=np.uint32)
    values = (packed.view(np.uint32)[..., None] >> shifts) & np.uint32(0xF)
    return values.astype(np.int32).reshape(*packed.shape[:-1], packed.shape[-1] * PACK_FACTOR)


def awq_pack(intweight: np.ndarray, zeros: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """pack.py:73-75."""
    return pack_int4(intweight), pack_int4(zeros)


def awq_unpack(qweight: np.ndarray) -> np.ndarray:
    """pack.py:78-80."""
    return unpack_int4(qweight)


def awq_quantize(weight: np.ndarray, group_size: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """pack.py:83-107: min-max asymmetric int4 in AWQ GEMM format, fp32 arithmetic,
    round-half-to-even. ``weight [N, K]`` -> ``(qweight [K, N/8], qzeros [K/G, N/8],
    scales [K/G, N] fp16)``."""
    n, k = weight.shape
    if k % group_size != 0:
        raise ValueError(f"K={k} is not a multiple of group_size={group_size}")
    w = np.asarray(weight, dtype=np.float32).reshape(n, k // group_size, group_size)
    max_val = w.max(axis=-1, keepdims=True)
    min_val = w.min(axis=-1, keepdims=True)
    scales = (np.maximum(max_val - min_val, np.float32(1e-5)) / np.float32(15)).astype(np.float16)
    scales = scales.astype(np.float32)
    zeros = np.clip(-np.rint(min_val / scales), 0, 15)
    q = np.clip(np.rint(w / scales) + zeros, 0, 15)
    intweight = q.reshape(n, k).T.astype(np.int32)
    zeros_kn = zeros[..., 0].T.astype(np.int32)
    scales_kn = scales[..., 0].T.astype(np.float16)
    qweight, qzeros = awq_pack(intweight, zeros_kn)
    return np.ascontiguousarray(qweight), np.ascontiguousarray(qzeros), np.ascontiguousarray(scales_kn)


def awq_dequantize(qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray, group_size: int) -> np.ndarray:
    """pack.py:110-117: ``fp16(q - z) * s`` as fp16 ``[K, N]`` (fp16 multiply, one rounding)."""
    q = awq_unpack(qweight)
    z = np.repeat(awq_unpack(qzeros), group_size, axis=0)
    s = np.repeat(np.asarray(scales, dtype=np.float16), group_size, axis=0)
    return (q - z).astype(np.float16) * s


@dataclass(frozen=True)
class W4A16Weights:
    """pack.py:123-138."""

    qweight_t: np.ndarray  # int32 [N, K // 8]
    scales: np.ndarray  # fp16 [K // G, N]
    qzeros: np.ndarray  # int32 [K // G, N // 8]
    group_size: int

    @property
    def n(self) -> int:
        return int(self.qweight_t.shape[0])

    @property
    def k(self) -> int:
        return int(self.qweight_t.shape[1]) * PACK_FACTOR


def repack_awq_to_tf(qweight: np.ndarray) -> np.ndarray:
    """pack.py:141-143: ``pack_int4(awq_unpack(qweight).T)``."""
    return np.ascontiguousarray(pack_int4(np.ascontiguousarray(awq_unpack(qweight).T)))


def repack_tf_to_awq(qweight_t: np.ndarray) -> np.ndarray:
    """pack.py:146-148."""
    return np.ascontiguousarray(pack_int4(np.ascontiguousarray(unpack_int4(qweight_t).T)))


def validate_awq(qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray, group_size: int) -> None:
    """pack.py:151-168 (same messages)."""
    if qweight.dtype != np.int32 or qzeros.dtype != np.int32:
        raise ValueError("qweight and qzeros must be int32")
    if scales.dtype != np.float16:
        raise ValueError(f"scales must be fp16, got {scales.dtype}")
    if group_size not in SUPPORTED_GROUP_SIZES:
        raise ValueError(f"group_size {group_size} not in {SUPPORTED_GROUP_SIZES}")
    k, n8 = qweight.shape
    n = n8 * PACK_FACTOR
    if k % group_size != 0:
        raise ValueError(f"K={k} is not a multiple of group_size={group_size}")
    if tuple(qzeros.shape) != (k // group_size, n8):
        raise ValueError(f"qzeros shape {tuple(qzeros.shape)} != {(k // group_size, n8)}")
    if tuple(scales.shape) != (k // group_size, n):
        raise ValueError(f"scales shape {tuple(scales.shape)} != {(k // group_size, n)}")


def pack_awq(qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray, group_size: int) -> W4A16Weights:
    """pack.py:171-181."""
    validate_awq(qweight, qzeros, scales, group_size)
    return W4A16Weights(
        qweight_t=repack_awq_to_tf(qweight),
        scales=np.ascontiguousarray(scales),
        qzeros=np.ascontiguousarray(qzeros),
        group_size=group_size,
    )


def unpack_to_awq(weights: W4A16Weights) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """pack.py:184-186."""
    return repack_tf_to_awq(weights.qweight_t), weights.qzeros, weights.scales


def dequantize_tf(weights: W4A16Weights) -> np.ndarray:
    """pack.py:189-194: TokenForge layout -> fp16 ``[N, K]``."""
    q = unpack_int4(weights.qweight_t)
    z = np.repeat(unpack_int4(weights.qzeros), weights.group_size, axis=0).T
    s = np.repeat(np.asarray(weights.scales, dtype=np.float16), weights.group_size, axis=0).T
    return (q - z).astype(np.float16) * s


# --------------------------------------------------------------------------- gfx950 tile layout
#
# The layout this build's pack_awq emits (no counterpart in the reference, whose pack_awq keeps
# the TokenForge layout above; the kernels' tokenforge_amd/csrc/tile_layout.h states the same
# maps). Rows come in tiles of 16 (t = n // 16, c = n % 16, r_t = min(16, N - 16 t)). qweight_t
# moves in 16-byte chunks (chunk q of row n = its words 4q..4q+3, K offsets 32q..32q+31):
#   chunk (n, q)  -> 16 t Q + 4 r_t (q // 4) + (q % 4) r_t + c       (Q = K / 32)
#   scale (p, n)  -> 16 t P + p r_t + c                               (P = K / G)
#   zero  (p, w)  -> 2 t P + p (r_t // 8) + (w - 2 t),  t = w // 2
# tile_order_* below define the same layout a second way, by the order in which a tile's
# 128-wide K steps, chunk columns and rows are laid down; the tests require both to agree.


def _tile_rows(n_total: int, t: np.ndarray) -> np.ndarray:
    return np.minimum(16, n_total - 16 * t)


def tile_chunk_index(n: np.ndarray, q: np.ndarray, n_total: int, q_total: int) -> np.ndarray:
    t, c = n // 16, n % 16
    rt = _tile_rows(n_total, t)
    return 16 * t * q_total + 4 * rt * (q // 4) + (q % 4) * rt + c


def tile_scale_index(p: np.ndarray, n: np.ndarray, n_total: int, p_total: int) -> np.ndarray:
    t = n // 16
    return 16 * t * p_total + p * _tile_rows(n_total, t) + n % 16


def tile_zero_index(p: np.ndarray, w: np.ndarray, n_total: int, p_total: int) -> np.ndarray:
    t = w // 2
    return 2 * t * p_total + p * (_tile_rows(n_total, t) // 8) + (w - 2 * t)


def tile_pack(
    qweight_t: np.ndarray, scales: np.ndarray, qzeros: np.ndarray, group_size: int
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """TokenForge-layout (qweight_t, scales, qzeros) -> the same tensors in the tile layout."""
    n, words = qweight_t.shape
    q_total, p_total = words // 4, (words * 8) // group_size
    chunks = np.ascontiguousarray(qweight_t).reshape(n, q_total, 4)
    nn, qq = np.meshgrid(np.arange(n), np.arange(q_total), indexing="ij")
    qw = np.empty((n * q_total, 4), dtype=np.int32)
    qw[tile_chunk_index(nn, qq, n, q_total).ravel()] = chunks.reshape(-1, 4)
    pp, ns = np.meshgrid(np.arange(p_total), np.arange(n), indexing="ij")
    sc = np.empty(p_total * n, dtype=np.float16)
    sc[tile_scale_index(pp, ns, n, p_total).ravel()] = np.asarray(scales).ravel()
    pz, wz = np.meshgrid(np.arange(p_total), np.arange(n // 8), indexing="ij")
    qz = np.empty(p_total * (n // 8), dtype=np.int32)
    qz[tile_zero_index(pz, wz, n, p_total).ravel()] = np.asarray(qzeros).ravel()
    return qw.reshape(n, words), sc.reshape(p_total, n), qz.reshape(p_total, n // 8)


def tile_unpack(
    qweight_tile: np.ndarray, scales_tile: np.ndarray, qzeros_tile: np.ndarray, group_size: int
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Inverse of :func:`tile_pack`."""
    n, words = qweight_tile.shape
    q_total, p_total = words // 4, (words * 8) // group_size
    nn, qq = np.meshgrid(np.arange(n), np.arange(q_total), indexing="ij")
    qw = np.ascontiguousarray(qweight_tile).reshape(-1, 4)[tile_chunk_index(nn, qq, n, q_total)]
    pp, ns = np.meshgrid(np.arange(p_total), np.arange(n), indexing="ij")
    sc = np.asarray(scales_tile).ravel()[tile_scale_index(pp, ns, n, p_total)]
    pz, wz = np.meshgrid(np.arange(p_total), np.arange(n // 8), indexing="ij")
    qz = np.asarray(qzeros_tile).ravel()[tile_zero_index(pz, wz, n, p_total)]
    return qw.reshape(n, words), sc.astype(np.float16), qz.astype(np.int32)


def tile_order_chunks(n_total: int, q_total: int) -> list[tuple[int, int]]:
    """(row, chunk) pairs in the order the tile layout stores them: tile by tile, 128-wide K
    step by step, chunk column g by g, row by row."""
    out = []
    for t in range((n_total + 15) // 16):
        rows = min(16, n_total - 16 * t)
        for j in range((q_total + 3) // 4):
            for g in range(min(4, q_total - 4 * j)):
                out += [(16 * t + c, 4 * j + g) for c in range(rows)]
    return out


def tile_order_scales(n_total: int, p_total: int) -> list[tuple[int, int]]:
    """(group, row) pairs in storage order: tile by tile, group by group, row by row."""
    out = []
    for t in range((n_total + 15) // 16):
        rows = min(16, n_total - 16 * t)
        for p in range(p_total):
            out += [(p, 16 * t + c) for c in range(rows)]
    return out


def tile_order_zeros(n_total: int, p_total: int) -> list[tuple[int, int]]:
    """(group, zero word) pairs in storage order: tile by tile, group by group, word by word."""
    out = []
    for t in range((n_total + 15) // 16):
        words = min(16, n_total - 16 * t) // 8
        for p in range(p_total):
            out += [(p, 2 * t + w) for w in range(words)]
    return out


def pack_awq_tiles(qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray, group_size: int) -> W4A16Weights:
    """This build's pack_awq: the reference's pack_awq (pack.py:171-181), then the tile layout."""
    w = pack_awq(qweight, qzeros, scales, group_size)
    qw, sc, qz = tile_pack(w.qweight_t, w.scales, w.qzeros, group_size)
    return W4A16Weights(qweight_t=qw, scales=sc, qzeros=qz, group_size=group_size)
