"""Every compiled kernel variant on its own seeded random case.

The code-path tests pick representative configs; this sweep runs every W4A16-capable entry
of ``VARIANTS`` (the library's table; the W4A8-only fp8 GEMM has its own sweep) once each, with the shape, group size, M, split_k, bias and epilogue drawn
from a generator seeded by the variant's index, against the fp64 oracle with the derived
tolerance and the normwise bound (and the fused epilogues against their unfused torch expressions, bit for bit).
N is sometimes ragged against the tile; K sometimes ends in a partial 128-wide step. The
W4A8 form of every variant (x as e4m3fn codes, decoded while staging or into the workspace)
must equal the W4A16 result on the decoded x bit for bit when the row scale is 1.
"""

from __future__ import annotations

import random

import pytest
import torch

from tests.numerics import cases
from tests.numerics.test_w4a16 import _assert_close
from tokenforge.kernels.config import VARIANTS, GemmConfig
from tokenforge.kernels.hip.w4a16 import w4a8_gemm_ex, w4a16_gemm, w4a16_gemm_ex

pytestmark = pytest.mark.gpu


def _case(index: int, variant: tuple) -> dict:  # type: ignore[type-arg]
    kernel, bm, bn, bk, warps, stages = variant
    rng = random.Random(1000 + index)
    if kernel == "gemm_mfma" and bk != 128:
        group = rng.choice([g for g in (32, 64, 128) if g >= bk and g % bk == 0])
    else:
        group = rng.choice((32, 64, 128))
    k = group * rng.randint(2, 8) if rng.random() < 0.5 else 128 * rng.randint(2, 6)
    k = max(k, group)
    n = 8 * rng.randint(8, 64)
    if rng.random() < 0.5:
        n = 16 * rng.randint(4, 32)  # a multiple of 16 (the SiLU*mul epilogue needs it)
    if kernel == "gemv_mfma" and bk == 512:
        # The stream form: N % 16 == 0 (N % 32 == 0 under SiLU*mul), K % 128 == 0 with a step
        # per wave, M <= block_m.
        n = 32 * rng.randint(2, 24) + (16 if rng.random() < 0.3 else 0)
        k = 128 * rng.randint(max(2, warps), max(2, warps) + 6)
    if kernel == "gemm_mfma" and bk == 128 and stages >= 6:
        # The wave-tile form: N % 16 == 0 and K % 128 == 0 (N ragged against its tile).
        n = 16 * rng.randint(4, 32)
        k = 128 * rng.randint(2, 6)
    if kernel == "gemv_dot" or (kernel == "gemv_mfma" and bk == 512):
        m = rng.randint(1, bm)
    elif kernel == "gemv_mfma":
        m = rng.randint(1, 2 * bm + 3)
    else:
        m = rng.randint(1, 2 * bm + 5)
    split = rng.choice((1, 2, 3)) if kernel == "gemm_mfma" else 1
    silu_ok = n % 32 == 0 if (kernel == "gemv_mfma" and bk == 512) else n % 16 == 0
    epilogue = rng.choice(("none", "none", "residual", "silu_mul")) if silu_ok else "none"
    return {"cfg": GemmConfig(kernel, bm, bn, bk, split, warps, stages), "group": group, "k": k, "n": n, "m": m,
            "bias": rng.random() < 0.5, "epilogue": epilogue, "seed": index}


# The W4A16-capable variants; the W4A8-only fp8 GEMM variants are swept against the exact
# W4A8 oracle in test_w4a8_fp8.py (every variant, four shapes, split-K 1 and 4).
W4A16_INDICES = [i for i, v in enumerate(VARIANTS) if v[0] != "gemm_fp8"]


@pytest.mark.parametrize("index", W4A16_INDICES)
def test_every_variant(index: int, device: torch.device) -> None:
    c = _case(index, VARIANTS[index])
    cfg, g, k, n, m = c["cfg"], c["group"], c["k"], c["n"], c["m"]
    w = cases.layer_weights(n, k, c["seed"], g)
    wd = cases.on_device(w, device)
    x = cases.activations(m, k, c["seed"])
    b = cases.bias(n, c["seed"]) if c["bias"] else None
    xd, bd = x.to(device), None if b is None else b.to(device)
    print(f"variant {index}: {cfg} k={k} n={n} m={m} g={g}", flush=True)
    try:
        y = w4a16_gemm(xd, wd.qweight_t, wd.scales, wd.qzeros, g, cfg, bd)
    except ValueError as e:
        # The only refusals a drawn case may meet: an LDS bound of the shared-x GEMV forms.
        assert "fit" in str(e), f"{cfg} k={k} n={n} m={m} g={g}: {e}"
        return
    _assert_close(y, x, w, b)
    if c["epilogue"] == "silu_mul":
        fused = w4a16_gemm_ex(xd, wd.qweight_t, wd.scales, wd.qzeros, g, cfg, bd, "silu_mul")
        assert torch.equal(fused, torch.nn.functional.silu(y[:, : n // 2]) * y[:, n // 2 :]), str(cfg)
    elif c["epilogue"] == "residual":
        r = cases.activations(m, n, c["seed"] + 1).to(device)
        fused = w4a16_gemm_ex(xd, wd.qweight_t, wd.scales, wd.qzeros, g, cfg, bd, "residual", r)
        assert torch.equal(fused, r + y), str(cfg)


@pytest.mark.parametrize("index", W4A16_INDICES)
def test_every_variant_w4a8_unit_scale(index: int, device: torch.device) -> None:
    c = _case(index, VARIANTS[index])
    cfg, g, k, n, m = c["cfg"], c["group"], c["k"], c["n"], c["m"]
    wd = cases.on_device(cases.layer_weights(n, k, c["seed"], g), device)
    b = cases.bias(n, c["seed"]).to(device) if c["bias"] else None
    gen = torch.Generator().manual_seed(5000 + index)
    codes = torch.randint(0, 256, (m, k), generator=gen, dtype=torch.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x38  # no NaN codes
    x8 = codes.to(device).view(torch.float8_e4m3fn)
    one = torch.ones(1, dtype=torch.float32, device=device)
    print(f"variant {index}: {cfg} k={k} n={n} m={m} g={g} (w4a8)", flush=True)
    try:
        y8 = w4a8_gemm_ex(x8, one, wd.qweight_t, wd.scales, wd.qzeros, g, cfg, b)
    except ValueError as e:
        assert "fit" in str(e), f"{cfg} k={k} n={n} m={m} g={g}: {e}"
        return
    y16 = w4a16_gemm(x8.to(torch.float16), wd.qweight_t, wd.scales, wd.qzeros, g, cfg, b)
    assert torch.equal(y8, y16), f"{cfg} k={k} n={n} m={m} g={g}"
