"""Linear shapes of the numerics suite, derived from each model's decoder dimensions.

A decoder layer has four quantized linears as an engine sees them at TP=1 (q/k/v fused,
gate/up fused): qkv ``hidden -> hidden + 2 * kv``, o ``hidden -> hidden``, gate_up
``hidden -> 2 * intermediate`` and down ``intermediate -> hidden``; ``n`` is the output
width and ``k`` the reduction length. Two synthetic layers add N that no tile width divides
(still a multiple of 8, as AWQ packing requires). The reference's suite holds the same shapes
(tests/numerics/shapes.py:16-35).

``TOKENFORGE_SHAPE_SUITE=full`` selects every shape and the long M list; the default quick
suite keeps the small model, the ragged layers and a few M values.
"""

from __future__ import annotations

import os
from typing import NamedTuple


class LinearShape(NamedTuple):
    model: str
    layer: str
    n: int
    k: int


# model -> (hidden, fused k+v width / 2, intermediate)
_DECODERS: dict[str, tuple[int, int, int]] = {
    "qwen2.5-0.5b": (896, 128, 4864),
    "qwen2.5-7b": (3584, 512, 18944),
}
_RAGGED: tuple[tuple[str, int, int], ...] = (("n_ragged_small", 200, 256), ("n_ragged", 1000, 1024))


def decoder_linears(model: str) -> list[LinearShape]:
    hidden, kv, inter = _DECODERS[model]
    widths = {
        "qkv_proj": (hidden + 2 * kv, hidden),
        "o_proj": (hidden, hidden),
        "gate_up_proj": (2 * inter, hidden),
        "down_proj": (hidden, inter),
    }
    return [LinearShape(model, layer, n, k) for layer, (n, k) in widths.items()]


def ragged_linears() -> list[LinearShape]:
    return [LinearShape("synthetic", layer, n, k) for layer, n, k in _RAGGED]


_M_FULL = (1, 2, 3, 4, 7, 8, 15, 16, 31, 32, 33, 64, 127, 128, 129, 256)
_M_QUICK = (1, 3, 8, 16, 31, 129)


def suite() -> str:
    """``quick`` unless ``TOKENFORGE_SHAPE_SUITE=full``."""
    return os.environ.get("TOKENFORGE_SHAPE_SUITE", "quick")


def linear_shapes() -> list[LinearShape]:
    models = list(_DECODERS) if suite() == "full" else ["qwen2.5-0.5b"]
    return [s for model in models for s in decoder_linears(model)] + ragged_linears()


def m_values() -> tuple[int, ...]:
    return _M_FULL if suite() == "full" else _M_QUICK
