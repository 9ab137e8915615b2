"""M buckets and launch configurations of the gfx950 W4A16 kernels.

Counterpart of the reference's ``config.py`` (config.py:8-117). Differences, each forced by
the hardware or by the single HIP path:

* ``M_BUCKETS`` runs up to 4096: every M, prefill included, is served by a HIP kernel chosen
  through the bucket's autotune entry (the reference sends M > 128 to dequant + cuBLAS).
* ``GemmConfig`` names a compiled kernel variant: ``kernel`` is one of ``KERNELS`` and the
  tuple ``(kernel, block_m, block_n, block_k, num_warps, num_stages)`` must be in
  ``VARIANTS`` (the table ``libtokenforge_hip.so`` exports; a CPU test keeps the two equal).
  ``split_k`` is a runtime value.

Field meaning per kernel family:

========== =========================== ================================================
kernel     block_m / block_n / block_k  split_k / num_warps / num_stages
========== =========================== ================================================
gemv_dot   max M (1,2,4) / columns per  1 / waves per workgroup / 128-wide K steps in
           workgroup (16*RT) / 128 or   flight per wave; block_k as for gemv_mfma
           256
gemv_mfma  M per tile (16,32) / columns 1 / waves per workgroup / 128-wide K steps in
           per workgroup (16*RT) / 128  flight per wave. block_k 128: the waves split
           or 256                       K over the same columns and add their partials
                                        on chip; block_k 256: the waves take different
                                        column sets (block_n each) over the whole K and
                                        share one staged x
gemv_mfma  max M (4) / 16 / 512: the    1 / waves per workgroup / steps in flight per wave.
(stream)   stream form                  Workgroups own tile ranges sized so the grid is
                                        resident; their waves take the range's 128-wide
                                        steps round robin (neighbouring blocks in flight)
gemm_mfma  LDS tile M / tile N / tile K K slices across workgroups (fp32 workspace,
                                        fixed-order reduce) / 4, 8 or 16 waves / 2: two
                                        LDS buffers, 3 and 4: pipelined with 2 and 3 x
                                        stages, 6 and 7: the same on 16x16 MFMA fragments
                                        (block_k 64); block_k 128: skinny form, num_stages
                                        = x stages (wave-tile form: 4 + x stages)
gemm_fp8   LDS tile M / tile N / 128    as gemm_mfma (8 waves, num_stages = x stages +
           (one group per block)        1). W4A8 only: e4m3 x on the fp8 MFMA, the group
                                        scale applied in fp32 after each group; chosen by
                                        ``fp8_gemm_config``, not by the W4A16 tuner
========== =========================== ================================================

Every kernel reads the weights in the gfx950 tile layout that ``pack.pack_awq`` produces.
"""

from __future__ import annotations

import functools
from dataclasses import asdict, dataclass, replace
from typing import Any

M_BUCKETS: tuple[int, ...] = (1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 1024, 2048, 4096)
MAX_BUCKET_M = M_BUCKETS[-1]
GEMV_MAX_M = 32
"""Largest bucket the streaming (gemv) kernels serve; by default larger ones use the GEMM."""
GEMM_MIN_M = 16
"""Smallest bucket the gemm_mfma kernels may serve (the tuner weighs both families at 16, 32)."""

KERNELS: tuple[str, ...] = ("gemv_dot", "gemv_mfma", "gemm_mfma", "gemm_fp8")
NUM_CUS = 256
"""MI355X compute units; the split heuristics aim to put several waves on each."""

_WAVES = (1, 2, 4, 8, 16)

# Compiled streaming variants: (kernel, block_m, column tiles RT, block_k, ring depth P, max
# waves). block_k = 128: the waves of a workgroup split K and x is staged in LDS per wave;
# block_k = 256: the waves take different column tiles over the whole K and share one copy of
# x. The wave cap keeps each variant within the VGPR budget of its launch bound (no spills).
GEMV_TEMPLATES: tuple[tuple[str, int, int, int, int, int], ...] = (
    ("gemv_dot", 1, 1, 128, 2, 16), ("gemv_dot", 1, 1, 128, 4, 16), ("gemv_dot", 1, 2, 128, 2, 16),
    ("gemv_dot", 2, 1, 128, 2, 16), ("gemv_dot", 4, 1, 128, 2, 16),
    ("gemv_dot", 1, 1, 256, 2, 8), ("gemv_dot", 1, 1, 256, 4, 8), ("gemv_dot", 2, 1, 256, 4, 8),
    ("gemv_dot", 4, 1, 256, 4, 8),
    ("gemv_mfma", 16, 1, 128, 2, 16), ("gemv_mfma", 16, 1, 128, 4, 16), ("gemv_mfma", 16, 1, 128, 8, 16),
    ("gemv_mfma", 16, 2, 128, 2, 16), ("gemv_mfma", 16, 2, 128, 4, 8), ("gemv_mfma", 16, 4, 128, 2, 8),
    ("gemv_mfma", 32, 1, 128, 2, 16), ("gemv_mfma", 32, 2, 128, 2, 8),
    ("gemv_mfma", 16, 1, 256, 2, 8), ("gemv_mfma", 16, 1, 256, 4, 8), ("gemv_mfma", 16, 1, 256, 8, 8),
    ("gemv_mfma", 16, 2, 256, 2, 8), ("gemv_mfma", 16, 2, 256, 4, 8), ("gemv_mfma", 32, 1, 256, 2, 8),
)


def _gemv_variants() -> list[tuple[str, int, int, int, int, int]]:
    out = []
    for kernel, bm, rt, bk, stages, max_waves in GEMV_TEMPLATES:
        out += [(kernel, bm, 16 * rt, bk, w, stages) for w in _WAVES if w <= max_waves]
    return out


STREAM_BLOCK_K = 512
"""``block_k`` of the GEMV stream form (gemv_mfma, M <= its block_m)."""
STREAM_MAX_M = 4
"""block_m of the stream form that serves M <= 4 (and runs the RMSNorm prologue)."""
STREAM_WIDE_M = 8
"""block_m of the stream form that serves the bucket of M = 5..8 (no RMSNorm prologue)."""
STREAM_MAX_X_BYTES = 96 * 1024
"""The stream form stages x in LDS: M rows of K + 8 fp16 values (of K / split_k + 8 under a K
split) must fit this."""
STREAM_SPLITS = (2, 4)
"""K splits the tuner tries on the stream form (split_k 1 besides): each workgroup stages and
multiplies one K slice, the split-K reduce adds the slices."""


def _stream_variants() -> list[tuple[str, int, int, int, int, int]]:
    # block_m 4: ring depth 2 and 4, every wave count; block_m 8: 4, 8 or 16 waves.
    return ([("gemv_mfma", STREAM_MAX_M, 16, STREAM_BLOCK_K, w, p) for p in (2, 4) for w in _WAVES]
            + [("gemv_mfma", STREAM_WIDE_M, 16, STREAM_BLOCK_K, w, p) for p in (2, 4) for w in (4, 8, 16)])


NORM_MAX_K = 8192
"""Largest K whose RMSNorm the GEMV stream form runs in its prologue."""


def norm_scratch_bytes(m: int, k: int) -> int:
    """LDS the stream form's RMSNorm prologue adds: M rows of chunk sums (fp64), each padded to
    the power of two >= K / 8 (at least 64), 256 bytes of maxima and the staged norm weight
    (K fp16)."""
    lpad = 64
    while lpad < k // 8:
        lpad *= 2
    return m * lpad * 8 + 256 + 2 * k


def stream_slice_k(k: int, split_k: int) -> int:
    """K of the longest slice when the stream form splits K over ``split_k`` workgroup sets."""
    return -(-(k // 128) // split_k) * 128


def stream_form_applies(m: int, n: int, k: int, num_warps: int, norm: bool = False,
                        max_m: int = STREAM_MAX_M, split_k: int = 1) -> bool:
    """Whether the op runs a call of this shape on the GEMV stream form when its bucket's config
    is that form (``max_m``: the config's block_m, ``split_k``: its K split): M <= max_m, N % 32
    == 0, K % 128 == 0 with at least one 128-wide step per wave in every K slice, and the
    slice of x small enough to stage in LDS. The rule does not depend on the epilogue, so a
    plain call and its fused SiLU*mul or residual twin run the same kernel and agree bit for bit
    (the library itself runs plain and residual calls on N % 16 == 0 as well). With ``norm``
    (the RMSNorm prologue of ``rmsnorm_fp8_w4a16_linear``, on the block_m 4 form without a K
    split only) M is at most 4, K at most NORM_MAX_K and the staged x plus the prologue's
    scratch must fit."""
    if k % 128 or split_k < 1:
        return False
    x_bytes = m * (stream_slice_k(k, split_k) + 8) * 2 + (norm_scratch_bytes(m, k) if norm else 0)
    return (
        1 <= m <= (STREAM_MAX_M if norm else max_m)
        and n % 32 == 0
        and (k // 128) // split_k >= num_warps
        and x_bytes <= STREAM_MAX_X_BYTES
        and (not norm or (k <= NORM_MAX_K and split_k == 1))
    )


NORM_FUSED_MAX_M = 1
"""``rmsnorm_fp8_w4a16_linear`` runs the norm inside the GEMV (its prologue) up to this M. Measured
on MI355X (qkv and gate_up of Qwen2.5-7B): at M = 1 the prologue saves the norm kernel's launch
(qkv 9.7 us against 7.3 + 3.5 for the two kernels); at M = 2 and 4 every workgroup's norm of
several rows takes longer than the separate norm kernel (qkv M = 4: 16.2 us against 11.6)."""
NORM_RING_DEPTH = 4
"""Ring depth (num_stages) of the stream form when it runs the RMSNorm prologue: the loads in
flight while the prologue runs keep HBM busy (qkv M = 1: 9.7 us at depth 4 against 10.5 at 2;
gate_up 19.9 against 21.3; depth 8 no better)."""


def norm_fused_config(cfg: GemmConfig, m: int, n: int, k: int) -> GemmConfig | None:
    """The config ``rmsnorm_fp8_w4a16_linear`` runs the fused kernel on, given the bucket's
    ``cfg``, or None where it runs the norm kernel and the linear: M <= NORM_FUSED_MAX_M, a
    stream-form config of block_m 4 without a K split, and the prologue fits
    (``stream_form_applies(norm=True)``); the ring deepened to NORM_RING_DEPTH. Both routes give
    the same bits."""
    if not (1 <= m <= NORM_FUSED_MAX_M and cfg.stream and cfg.block_m == STREAM_MAX_M and cfg.split_k == 1):
        return None
    if not stream_form_applies(m, n, k, cfg.num_warps, norm=True):
        return None
    return replace(cfg, num_stages=max(cfg.num_stages, NORM_RING_DEPTH))


def _gemm_variants() -> list[tuple[str, int, int, int, int, int]]:
    # num_stages 2: two LDS buffers, operands staged through registers (any group size).
    tiles = [(64, 64, 64), (64, 128, 64), (128, 64, 64), (128, 128, 64), (128, 256, 64),
             (256, 128, 64), (256, 256, 64), (64, 64, 32), (128, 128, 32), (256, 128, 32)]
    out = [("gemm_mfma", bm, bn, bk, 4, 2) for bm, bn, bk in tiles]
    # num_stages 3 / 4: pipelined form, x streamed into 2 / 3 LDS stages, weights prefetched two
    # blocks ahead (block_k 64, group size 64 or 128); 4 or 8 waves.
    tiles3 = [(256, 160), (256, 128), (128, 256), (128, 128), (256, 192), (256, 96), (64, 256), (128, 192)]
    out += [("gemm_mfma", bm, bn, 64, 4, 4) for bm, bn in tiles3]
    out += [("gemm_mfma", 256, 256, 64, 8, 3), ("gemm_mfma", 256, 192, 64, 8, 3),
            ("gemm_mfma", 256, 192, 64, 8, 4), ("gemm_mfma", 256, 128, 64, 8, 3),
            ("gemm_mfma", 128, 256, 64, 8, 3), ("gemm_mfma", 256, 160, 64, 8, 3)]
    # ... and 16 waves (four per SIMD), 32-row wave tiles.
    out += [("gemm_mfma", 256, 192, 64, 16, 3), ("gemm_mfma", 256, 192, 64, 16, 4), ("gemm_mfma", 256, 128, 64, 16, 3)]
    # num_stages 6 / 7: the same pipeline on 16x16 MFMA fragments (16-column wave-tile
    # granularity): 256 x 160 tiles with 16 or 8 waves, 256 x 128 .. 256 with 8, 128-row tiles
    # with 4 or 8.
    out += [("gemm_mfma", 256, 160, 64, 16, 6), ("gemm_mfma", 256, 160, 64, 16, 7), ("gemm_mfma", 256, 160, 64, 8, 6),
            ("gemm_mfma", 256, 160, 64, 8, 7), ("gemm_mfma", 256, 192, 64, 8, 6), ("gemm_mfma", 256, 224, 64, 8, 6),
            ("gemm_mfma", 256, 128, 64, 8, 6), ("gemm_mfma", 256, 256, 64, 8, 6), ("gemm_mfma", 128, 160, 64, 4, 6),
            ("gemm_mfma", 128, 128, 64, 4, 6), ("gemm_mfma", 128, 256, 64, 8, 6)]
    # num_stages 8: the producer / consumer form (two x stages): num_warps consumer waves only
    # read fragments and run MFMAs, four producer waves stage x and dequantize the weights.
    out += [("gemm_mfma", 256, 160, 64, 8, 8), ("gemm_mfma", 256, 128, 64, 8, 8), ("gemm_mfma", 128, 256, 64, 8, 8),
            ("gemm_mfma", 128, 128, 64, 4, 8), ("gemm_mfma", 256, 192, 64, 8, 8)]
    # block_k 128: skinny form (M <= 128), weights streamed into MFMA registers, 4 waves,
    # num_stages = x stages in LDS.
    skinny = [(1, 1, 3), (1, 2, 3), (1, 4, 3), (2, 1, 3), (2, 2, 3), (2, 4, 3), (4, 1, 3), (4, 2, 3),
              (4, 4, 3), (8, 1, 3), (8, 2, 3), (2, 2, 2), (4, 2, 2)]
    out += [("gemm_mfma", 16 * mt, 64 * rt, 128, 4, st) for mt, rt, st in skinny]
    # ... and with two waves along M: 256 x 160 tiles (gate_up at M >= 256: 237 tiles).
    out += [("gemm_mfma", 256, 160, 128, 4, 2)]
    # block_k 128, num_stages 4 + S: the wave-tile form (one wave per SIMD, 16 MT x 16 RT per
    # wave, WM waves along M), S x stages (x issued S - 1 steps ahead, weights three).
    wave_tiles = [(8, 5, 1, 3), (8, 4, 1, 4), (8, 3, 1, 4), (8, 2, 1, 4)]
    out += [("gemm_mfma", 16 * mt * wm, 16 * rt * (4 // wm), 128, 4, 4 + st) for mt, rt, wm, st in wave_tiles]
    return out


# W4A8 fp8 GEMM tiles (block_m, block_n, waves along M, waves along N, x stages), in the
# library's order.
FP8_TILES: tuple[tuple[int, int, int, int, int], ...] = (
    (256, 192, 4, 2, 2), (256, 128, 4, 2, 2), (128, 256, 2, 4, 2), (256, 160, 4, 2, 2), (128, 128, 2, 4, 2),
    (256, 192, 4, 2, 3),
)


FP8_PC_TILES: tuple[tuple[int, int, int, int], ...] = ((256, 160, 4, 2), (256, 128, 4, 2), (128, 256, 2, 4), (128, 128, 2, 4))
"""The fp8 GEMM's producer / consumer form (num_stages 8): (block_m, block_n, consumer waves
along M, along N), in the library's order after FP8_TILES."""


def _fp8_variants() -> list[tuple[str, int, int, int, int, int]]:
    return ([("gemm_fp8", bm, bn, 128, wm * wn, s + 1) for bm, bn, wm, wn, s in FP8_TILES]
            + [("gemm_fp8", bm, bn, 128, wm * wn, 8) for bm, bn, wm, wn in FP8_PC_TILES])


VARIANTS: tuple[tuple[str, int, int, int, int, int], ...] = tuple(
    _gemv_variants() + _stream_variants() + _gemm_variants() + _fp8_variants()
)
"""(kernel, block_m, block_n, block_k, num_warps, num_stages), in the library's order."""
_VARIANT_SET = frozenset(VARIANTS)


def m_bucket(m: int) -> int:
    """Smallest bucket >= m (config.py:13-20). M above the largest bucket uses the largest."""
    if m < 1:
        raise ValueError(f"M must be >= 1, got {m}")
    for b in M_BUCKETS:
        if m <= b:
            return b
    raise ValueError(f"M={m} exceeds the largest bucket ({MAX_BUCKET_M})")


def family_for_bucket(bucket: int) -> str:
    """Default family of a bucket: ``gemv`` below GEMM_MIN_M, ``gemm`` from it on (the tuner
    may still pick a gemv kernel up to GEMV_MAX_M)."""
    return "gemv" if bucket < GEMM_MIN_M else "gemm"


@dataclass(frozen=True)
class GemmConfig:
    kernel: str
    block_m: int
    block_n: int
    block_k: int
    split_k: int = 1
    num_warps: int = 4
    num_stages: int = 2

    @property
    def path(self) -> str:
        return self.kernel

    @property
    def skinny(self) -> bool:
        """The skinny gemm_mfma form (block_k 128), which reads each lane's group itself."""
        return self.kernel == "gemm_mfma" and self.block_k == 128

    @property
    def stream(self) -> bool:
        """The GEMV stream form (gemv_mfma, block_k 512), which serves M <= 4."""
        return self.kernel == "gemv_mfma" and self.block_k == STREAM_BLOCK_K

    @property
    def family(self) -> str:
        return "gemm" if self.kernel in ("gemm_mfma", "gemm_fp8") else "gemv"

    def variant(self) -> tuple[str, int, int, int, int, int]:
        return (self.kernel, self.block_m, self.block_n, self.block_k, self.num_warps, self.num_stages)

    def validate(self, group_size: int) -> None:
        """Raise ``ValueError`` if this config cannot run for ``group_size``."""
        if self.kernel not in KERNELS:
            raise ValueError(f"kernel={self.kernel!r} not in {KERNELS}")
        if self.kernel == "gemm_mfma" and not self.skinny and (
            self.block_k <= 0 or self.block_k > group_size or group_size % self.block_k
        ):
            raise ValueError(f"block_k={self.block_k} must divide group_size={group_size}")
        if not 1 <= self.split_k <= 16:
            raise ValueError(f"split_k={self.split_k} must be in [1, 16]")
        if self.family != "gemm" and not self.stream and self.split_k != 1:
            raise ValueError(
                f"split_k={self.split_k}: {self.kernel} splits K across its num_warps waves; "
                "split_k must be 1"
            )
        if self.num_warps not in _WAVES:
            raise ValueError(f"num_warps={self.num_warps} must be a power of two <= 16")
        if not 1 <= self.num_stages <= 8:
            raise ValueError(f"num_stages={self.num_stages} must be in [1, 8]")
        if self.variant() not in _VARIANT_SET:
            raise ValueError(f"{self.variant()} is not a compiled variant (block_m/block_n/block_k)")

    def fits_bucket(self, bucket: int) -> bool:
        """Whether this config may serve M values of ``bucket`` (cache validation): the gemv
        kernels serve buckets up to GEMV_MAX_M (gemv_dot and the stream form only up to their
        block_m), gemm_mfma buckets from GEMM_MIN_M on."""
        if self.family == "gemm":
            return bucket >= GEMM_MIN_M
        if bucket > GEMV_MAX_M:
            return False
        if self.stream:  # block_m 4 serves buckets up to 4, block_m 8 the bucket above
            return bucket <= self.block_m and (self.block_m == STREAM_MAX_M or bucket > STREAM_MAX_M)
        return self.kernel != "gemv_dot" or self.block_m >= bucket

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)

    @classmethod
    def from_dict(cls, d: Any) -> GemmConfig:
        if not isinstance(d, dict):
            raise TypeError(f"config must be an object, got {type(d).__name__}")
        fields = set(cls.__dataclass_fields__)
        unknown = set(d) - fields
        if unknown:
            raise ValueError(f"unknown config keys {sorted(unknown)}")
        if not isinstance(d.get("kernel"), str):
            raise TypeError("config 'kernel' must be a string")
        ints = {k: v for k, v in d.items() if k != "kernel"}
        if not all(isinstance(v, int) and not isinstance(v, bool) for v in ints.values()):
            raise TypeError("config values must be integers")
        return cls(**d)


def _pow2_at_most(v: int, cap: int) -> int:
    p = 1
    while p * 2 <= min(v, cap):
        p *= 2
    return p


def split_k_gemv_config(n: int, k: int) -> GemmConfig:
    """The GEMV form that runs every shape (K split over the waves of a workgroup): one
    workgroup per 32 output columns, waves added until the grid holds about 12 per CU, never
    more waves than 128-wide K steps."""
    tiles = -(-n // 32)
    k_steps = max(1, -(-k // 128))
    waves = _pow2_at_most(max(1, -(-(12 * NUM_CUS) // tiles)), min(16, k_steps))
    return GemmConfig("gemv_mfma", 16, 32, 128, 1, waves, 2)


def default_config(bucket: int, n: int, k: int, group_size: int) -> GemmConfig:
    """Heuristic config used before tuning (config.py:71-92, re-derived for 256 CUs).

    Streaming kernels (M < 16): for M <= 4 the stream form with 8 waves and a ring of 2 where
    it applies; otherwise one workgroup per 32 output columns, adding
    waves (on-chip K slices) until the grid holds about 12 waves per CU, never more waves than
    128-wide K steps.
    Skinny GEMM (16 <= M <= 128): 16-64 rows x 64 or 128 columns per workgroup, K split until
    the grid holds about 1.5 workgroups per CU.
    Pipelined GEMM (M >= 256, group >= 64): 256 x 192 tiles of 8 waves (256 x 256 from M 1024);
    two-buffer GEMM for group 32.
    """
    if family_for_bucket(bucket) == "gemv":
        if bucket <= STREAM_MAX_M and stream_form_applies(bucket, n, k, 8):
            return GemmConfig("gemv_mfma", STREAM_MAX_M, 16, STREAM_BLOCK_K, 1, 8, 2)
        return split_k_gemv_config(n, k)
    if bucket <= 128:
        bm = min(bucket, 64)
        bn = 64 if bucket <= 64 else 128
        tiles = -(-n // bn) * -(-bucket // bm)
        k_steps = max(1, -(-k // 128))
        split = 1
        while tiles * split * 2 <= 3 * NUM_CUS and split * 2 <= min(8, k_steps):
            split *= 2
        return GemmConfig("gemm_mfma", bm, bn, 128, split, 4, 3)
    if group_size >= 64:
        bm, bn = (256, 192) if bucket <= 512 else (256, 256)
        tiles = -(-n // bn) * -(-bucket // bm)
        k_blocks = k // 64
        split = 1
        while tiles * split < NUM_CUS and split * 2 <= min(8, k_blocks):
            split *= 2
        return GemmConfig("gemm_mfma", bm, bn, 64, split, 8, 3)
    block_k = 64 if group_size >= 64 else 32
    if bucket <= 64:
        bm, bn = 64, 64
    elif bucket <= 128:
        bm, bn = 128, 128
    else:
        bm, bn = (256, 128) if block_k == 64 else (256, 128)
    tiles = -(-n // bn) * -(-bucket // bm)
    k_blocks = k // block_k
    split = 1
    while tiles * split < NUM_CUS and split * 2 <= min(16, k_blocks):
        split *= 2
    return GemmConfig("gemm_mfma", bm, bn, block_k, split, 4, 2)


def candidate_configs(bucket: int, group_size: int) -> list[GemmConfig]:
    """Autotune search space for one bucket: every compiled variant that fits the bucket (both
    families for buckets GEMM_MIN_M..GEMV_MAX_M)."""
    out: list[GemmConfig] = []
    for kernel, bm, bn, bk, warps, stages in VARIANTS:
        if kernel == "gemm_fp8":  # W4A8 only (fp8_gemm_config), never a W4A16 candidate
            continue
        cfg = GemmConfig(kernel, bm, bn, bk, 1, warps, stages)
        if not cfg.fits_bucket(bucket):
            continue
        if cfg.family == "gemv":
            if kernel == "gemv_mfma" and bm > 16 and bucket <= 16:
                continue
            out.append(cfg)
            if cfg.stream:  # K split across workgroups: x rows of a long K staged by slices
                out.extend(replace(cfg, split_k=s) for s in STREAM_SPLITS)
            continue
        if bk != 128 and (bk > group_size or group_size % bk):
            continue
        if bm > 2 * bucket:
            continue
        out.extend(GemmConfig(kernel, bm, bn, bk, s, warps, stages) for s in (1, 2, 4, 8))
    return out


def fill_split(cfg: GemmConfig, m: int, n: int, k: int, cus: int = 256) -> int:
    """The K split that finishes an LDS-tile GEMM launch in the fewest K blocks per CU when its
    workgroups run in whole rounds over ``cus`` CUs: argmin over s of ceil(tiles * s / cus) *
    ceil(blocks / s), the smallest such s. E.g. down_proj (3584 x 18944) at M = 256 in 256 x 128
    tiles: 28 tiles, 296 blocks of 64, split 9 (252 workgroups, 33 blocks each) against split
    8's 37 blocks. s stays within 16, the K blocks, and K / (8 M): the fp32 partials (s * M * N *
    4 bytes, written and read back) are then no larger than the packed weights (N * K / 2), the
    traffic the split is meant to spread. The tuner times the candidate like any other."""
    tiles = -(-m // cfg.block_m) * -(-n // cfg.block_n)
    blocks = k // cfg.block_k
    best, best_cost = 1, None
    for s in range(1, max(1, min(16, blocks, k // (8 * m))) + 1):
        cost = -(-tiles * s // cus) * -(-blocks // s)
        if best_cost is None or cost < best_cost:
            best, best_cost = s, cost
    return best


def fill_split_candidates(cands: list[GemmConfig], bucket: int, n: int, k: int, cus: int = 256) -> list[GemmConfig]:
    """For every LDS-tile GEMM tile among ``cands``, its :func:`fill_split` config when the
    candidates do not already hold it (they split K in powers of two)."""
    have = {(c.kernel, c.block_m, c.block_n, c.block_k, c.num_warps, c.num_stages, c.split_k) for c in cands}
    out: list[GemmConfig] = []
    for c in cands:
        if c.kernel != "gemm_mfma" or c.skinny or c.split_k != 1:
            continue
        s = fill_split(c, bucket, n, k, cus)
        key = (c.kernel, c.block_m, c.block_n, c.block_k, c.num_warps, c.num_stages, s)
        if key not in have:
            have.add(key)
            out.append(replace(c, split_k=s))
    return out


FP8_MIN_BUCKET = 128
"""W4A8 calls from this M bucket on run the fp8 GEMM (where it applies); smaller M stay on the
kernels that read the weights once per call (GEMV, skinny GEMM), which decode the codes to fp16."""


def fp8_gemm_applies(bucket: int, n: int, k: int, group_size: int) -> bool:
    """Whether a W4A8 call of this shape runs on the fp8 GEMM: prefill M, group_size 128,
    K % 128 == 0 and N % 16 == 0 (what ``gemm_fp8`` requires)."""
    return bucket >= FP8_MIN_BUCKET and group_size == 128 and k % 128 == 0 and n % 16 == 0


# Makespan model of the fp8 GEMM on MI355X (fit to its measured times on the Qwen2.5-7B shapes):
# a workgroup runs one 128-K block of a BM x BN tile at about 4.2 TFLOP/s, the 256 x 160 tile 5%
# slower per FLOP; a K split adds about 3 us plus its fp32 partials (split * M * N * 4 bytes
# written and read back) at about 4 TB/s.
_FP8_CU_FLOP_PER_US = 4.2e6
_FP8_SPLIT_US = 3.0
_FP8_PARTIAL_BYTES_PER_US = 4.0e6


@functools.lru_cache(maxsize=None)
def fp8_gemm_config(bucket: int, n: int, k: int) -> GemmConfig:
    """Launch config of the W4A8 fp8 GEMM for one bucket: the tile and K split with the lowest
    modelled time (rounds of workgroups over the CUs x blocks per workgroup x block time, plus
    the split's partials), in its producer / consumer form where the tile has one. On the
    Qwen2.5-7B shapes it picks the configs measured fastest: gate_up 256 x 160 at M = 256 and
    256 x 128 above; down 256 x 128 with split 9 / 2 / 1 at M = 256 / 1024 / 4096."""
    tiles_by_m = ((256, 128), (256, 160), (256, 192)) if bucket >= 256 else ((128, 256), (128, 128))
    k_blocks = max(1, k // 128)
    best: tuple[float, int, int, int] | None = None
    for bm, bn in tiles_by_m:
        tiles = -(-n // bn) * -(-bucket // bm)
        block_us = bm * bn * 128 * 2 / _FP8_CU_FLOP_PER_US * (1.05 if bn == 160 else 1.0)
        # Powers of two, and the split that fills the CUs in whole rounds (fill_split; with
        # 28 column tiles of down_proj, split 9 is 3% faster than 8 at M = 128 and 256).
        fill = fill_split(GemmConfig("gemm_fp8", bm, bn, 128, 1, 8, 3), bucket, n, k, NUM_CUS)
        for split in sorted({1, 2, 4, 8, fill}):
            if split > 1 and split * 4 > k_blocks:
                break
            rounds = -(-tiles * split // NUM_CUS)
            us = rounds * -(-k_blocks // split) * block_us
            if split > 1:
                us += _FP8_SPLIT_US + split * bucket * n * 8 / _FP8_PARTIAL_BYTES_PER_US
            if best is None or us < best[0]:
                best = (us, bm, bn, split)
    assert best is not None
    _, bm, bn, split = best
    # the producer / consumer form where the tile has one (same box, Qwen2.5-7B shapes: 3-14%
    # faster than the shared-role form at M = 256..4096)
    stages = 8 if any((bm, bn) == (pbm, pbn) for pbm, pbn, _, _ in FP8_PC_TILES) else 3
    return GemmConfig("gemm_fp8", bm, bn, 128, split, 8, stages)
