"""Which layer shapes and batch sizes the numerics suite runs.

Shapes come from each model's decoder dimensions, as an engine sees its four quantized linears
at TP=1 (q/k/v fused, gate/up fused): qkv maps ``hidden -> hidden + 2 * kv``, o
``hidden -> hidden``, gate_up ``hidden -> 2 * intermediate`` and down ``intermediate -> hidden``
(``n`` = output width, ``k`` = reduction length). Two synthetic layers have an N that no tile
width divides (still a multiple of 8, as AWQ packing needs). The table equals the reference's
suite (tests/numerics/shapes.py:16-35).

Two suites: ``quick`` (the default: the small model, the ragged layers, six M values) and
``full`` (both models and the long M list), chosen by ``TOKENFORGE_SHAPE_SUITE``.
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from typing import NamedTuple

SUITE_ENV = "TOKENFORGE_SHAPE_SUITE"


class LinearShape(NamedTuple):
    model: str
    layer: str
    n: int
    k: int


@dataclass(frozen=True)
class Decoder:
    """A decoder's widths: hidden size, the K (= V) projection width, the MLP width."""

    model: str
    hidden: int
    kv: int
    intermediate: int

    def linears(self) -> list[LinearShape]:
        h, kv, i = self.hidden, self.kv, self.intermediate
        return [
            LinearShape(self.model, "qkv_proj", h + 2 * kv, h),
            LinearShape(self.model, "o_proj", h, h),
            LinearShape(self.model, "gate_up_proj", 2 * i, h),
            LinearShape(self.model, "down_proj", h, i),
        ]


QWEN25_05B = Decoder("qwen2.5-0.5b", 896, 128, 4864)
QWEN25_7B = Decoder("qwen2.5-7b", 3584, 512, 18944)
RAGGED = (LinearShape("synthetic", "n_ragged_small", 200, 256), LinearShape("synthetic", "n_ragged", 1000, 1024))


@dataclass(frozen=True)
class ShapeSuite:
    name: str
    decoders: tuple[Decoder, ...]
    m_values: tuple[int, ...]

    @property
    def shapes(self) -> list[LinearShape]:
        return [s for d in self.decoders for s in d.linears()] + list(RAGGED)


SUITES = {
    "quick": ShapeSuite("quick", (QWEN25_05B,), (1, 3, 8, 16, 31, 129)),
    "full": ShapeSuite("full", (QWEN25_05B, QWEN25_7B), (1, 2, 3, 4, 7, 8, 15, 16, 31, 32, 33, 64, 127, 128, 129, 256)),
}


def active() -> ShapeSuite:
    """The suite ``TOKENFORGE_SHAPE_SUITE`` names ("full"), else the quick one."""
    return SUITES["full"] if os.environ.get(SUITE_ENV) == "full" else SUITES["quick"]
