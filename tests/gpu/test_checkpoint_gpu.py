"""GPU side of the AWQ checkpoint loader: a checkpoint quantized by the oracle's AWQ
quantizer (pack.py:83-107 restated), read, fused, repacked on the GPU and tuned into a fresh
cache; the repacked tensors equal the oracle repack of the fused AWQ tensors bit for bit, the
cache holds every shape and bucket, and the op on the loaded weights matches the oracle."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import tokenforge.kernels.ops  # noqa: F401  (registers torch.ops.tokenforge)
from oracle import pack as opack
from oracle import reference as oref
from tests.numerics.tolerance import NORMWISE_MAX, contract, relative_max_error
from tokenforge.kernels import autotune
from tokenforge.kernels import checkpoint as ck

pytestmark = pytest.mark.gpu
G = 128
H, KV, INTER = 512, 128, 768
LINEARS = {
    "self_attn.q_proj": (H, H),
    "self_attn.k_proj": (KV, H),
    "self_attn.v_proj": (KV, H),
    "self_attn.o_proj": (H, H),
    "mlp.gate_proj": (INTER, H),
    "mlp.up_proj": (INTER, H),
    "mlp.down_proj": (H, INTER),
}


def _write(d: Path) -> dict[str, np.ndarray]:
    tensors: dict[str, torch.Tensor] = {}
    awq: dict[str, np.ndarray] = {}
    for li in range(2):
        for j, (name, (n, k)) in enumerate(LINEARS.items()):
            gen = torch.Generator().manual_seed(1000 * li + j)
            w = (torch.randn((n, k), generator=gen) * 0.02).numpy()
            qweight, qzeros, scales = opack.awq_quantize(w, G)
            prefix = f"model.layers.{li}.{name}"
            for part, arr in (("qweight", qweight), ("qzeros", qzeros), ("scales", scales)):
                tensors[f"{prefix}.{part}"] = torch.from_numpy(arr)
                awq[f"{prefix}.{part}"] = arr
            if name.endswith(("q_proj", "k_proj", "v_proj")):
                b = (torch.randn((n,), generator=gen) * 0.1).to(torch.float16)
                tensors[f"{prefix}.bias"] = b
                awq[f"{prefix}.bias"] = b.numpy()
    d.mkdir(parents=True, exist_ok=True)
    save_file(tensors, str(d / "model.safetensors"))
    (d / "config.json").write_text(json.dumps({"quantization_config": {
        "quant_method": "awq", "bits": 4, "group_size": G, "zero_point": True, "version": "gemm"}}))
    return awq


def test_load_repack_tune_and_run(tmp_path: Path, monkeypatch: pytest.MonkeyPatch, device: torch.device) -> None:
    monkeypatch.setenv(autotune.CACHE_DIR_ENV, str(tmp_path / "cache"))
    awq = _write(tmp_path / "ckpt")
    loaded = ck.load_awq_checkpoint(tmp_path / "ckpt", device=device, tune_buckets=(1, 32))
    assert loaded.group_size == G and not loaded.fallbacks
    fused = {"self_attn.qkv_proj": ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"],
             "self_attn.o_proj": ["self_attn.o_proj"],
             "mlp.gate_up_proj": ["mlp.gate_proj", "mlp.up_proj"],
             "mlp.down_proj": ["mlp.down_proj"]}
    assert sorted(loaded.layers) == sorted(f"model.layers.{li}.{f}" for li in range(2) for f in fused)
    for li in range(2):
        for name, parts in fused.items():
            w, bias = loaded.layers[f"model.layers.{li}.{name}"]
            cat = {p: np.concatenate([awq[f"model.layers.{li}.{q}.{p}"] for q in parts], axis=1)
                   for p in ("qweight", "qzeros", "scales")}
            ref = opack.pack_awq(cat["qweight"], cat["qzeros"], cat["scales"], G)
            tiled = opack.pack_awq_tiles(cat["qweight"], cat["qzeros"], cat["scales"], G)
            assert np.array_equal(w.qweight_t.cpu().numpy(), tiled.qweight_t)
            assert np.array_equal(w.scales.cpu().numpy(), tiled.scales)
            assert np.array_equal(w.qzeros.cpu().numpy(), tiled.qzeros)
            b_ref = None
            if name == "self_attn.qkv_proj":
                b_ref = np.concatenate([awq[f"model.layers.{li}.{q}.bias"] for q in parts])
                assert np.array_equal(bias.cpu().numpy(), b_ref)
            else:
                assert bias is None
            gen = torch.Generator().manual_seed(li)
            x = torch.randn((5, w.k), generator=gen).to(torch.float16)
            y = torch.ops.tokenforge.w4a16_linear(x.to(device), w.qweight_t, w.scales, w.qzeros, bias, G, "hip")
            y64 = y.cpu().numpy().astype(np.float64)
            xr = x.numpy()
            r64 = oref.w4a16_reference(xr, ref, b_ref)
            # The derived bound plus half an fp16 ulp of each output: the result is rounded to
            # fp16 once, which the bound (made for |y| of order 1) does not cover at |y| ~ 10.
            half_ulp = np.spacing(np.abs(r64).astype(np.float16)).astype(np.float64) / 2
            excess = np.abs(y64 - r64) - half_ulp
            assert float(excess.max()) <= contract("cuda").atol(xr, opack.dequantize_tf(ref))
            assert relative_max_error(y64, oref.w4a16_fp32(xr, ref, b_ref)) <= NORMWISE_MAX
    shapes = {(w.n, w.k) for w, _ in loaded.layers.values()}
    assert set(loaded.tuned) == shapes
    cache = list((tmp_path / "cache").glob("*.json"))
    assert len(cache) == 1
    entries = json.loads(cache[0].read_text())
    text = json.dumps(entries)
    for n, k in shapes:
        for bucket in (1, 32):
            assert f'"{bucket}:{n}:{k}:{G}"' in text
