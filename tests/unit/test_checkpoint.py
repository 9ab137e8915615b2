"""Host side of the AWQ checkpoint loader: config parsing, shard discovery, grouping, fusion
along N, and the errors for malformed checkpoints (the GPU repack and tuning are covered by
tests/gpu/test_checkpoint_gpu.py)."""

from __future__ import annotations

import json
from pathlib import Path

import pytest
import torch
from safetensors.torch import save_file

from tokenforge.kernels import checkpoint as ck
from tokenforge.kernels.dispatch import HipUnavailableError

G = 128
H, KV, INTER = 256, 64, 384
LINEARS = {  # name -> (N, K)
    "self_attn.q_proj": (H, H),
    "self_attn.k_proj": (KV, H),
    "self_attn.v_proj": (KV, H),
    "self_attn.o_proj": (H, H),
    "mlp.gate_proj": (INTER, H),
    "mlp.up_proj": (INTER, H),
    "mlp.down_proj": (H, INTER),
}
QUANT = {"quant_method": "awq", "bits": 4, "group_size": G, "zero_point": True, "version": "gemm"}


def awq_tensors(n: int, k: int, seed: int, bias: bool) -> dict[str, torch.Tensor]:
    gen = torch.Generator().manual_seed(seed)
    t = {
        "qweight": torch.randint(-(2**31), 2**31 - 1, (k, n // 8), generator=gen, dtype=torch.int32),
        "qzeros": torch.randint(-(2**31), 2**31 - 1, (k // G, n // 8), generator=gen, dtype=torch.int32),
        "scales": (torch.rand((k // G, n), generator=gen) * 9e-3 + 1e-3).to(torch.float16),
    }
    if bias:
        t["bias"] = torch.randn((n,), generator=gen).to(torch.float16)
    return t


def write_checkpoint(d: Path, layers: int = 2, shards: int = 1, quant: dict | None = QUANT) -> dict[str, torch.Tensor]:
    tensors: dict[str, torch.Tensor] = {}
    for li in range(layers):
        for j, (name, (n, k)) in enumerate(LINEARS.items()):
            for part, t in awq_tensors(n, k, 100 * li + j, bias=name.split(".")[-1] in ("q_proj", "k_proj", "v_proj")).items():
                tensors[f"model.layers.{li}.{name}.{part}"] = t
        tensors[f"model.layers.{li}.input_layernorm.weight"] = torch.ones(H, dtype=torch.float16)
    tensors["lm_head.weight"] = torch.zeros((8, H), dtype=torch.float16)
    d.mkdir(parents=True, exist_ok=True)
    keys = sorted(tensors)
    if shards == 1:
        save_file(tensors, str(d / "model.safetensors"))
    else:
        weight_map = {}
        for s in range(shards):
            part = {k: tensors[k] for k in keys[s::shards]}
            fname = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
            save_file(part, str(d / fname))
            weight_map.update({k: fname for k in part})
        (d / ck.INDEX_FILE).write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    cfg = {"model_type": "qwen2"}
    if quant is not None:
        cfg["quantization_config"] = quant
    (d / "config.json").write_text(json.dumps(cfg))
    return tensors


def test_quant_config(tmp_path: Path) -> None:
    write_checkpoint(tmp_path)
    assert ck.read_quant_config(tmp_path) == ck.QuantConfig(4, G, True, "gemm")
    assert ck.read_quant_config(tmp_path / "model.safetensors") == ck.QuantConfig(4, G, True, "gemm")


@pytest.mark.parametrize(
    ("quant", "match"),
    [
        ({**QUANT, "quant_method": "gptq"}, "not AWQ"),
        ({**QUANT, "bits": 8}, "8-bit"),
        ({**QUANT, "zero_point": False}, "zero points"),
        ({**QUANT, "version": "gemv"}, "GEMM layout"),
    ],
)
def test_quant_config_rejects(tmp_path: Path, quant: dict, match: str) -> None:  # type: ignore[type-arg]
    write_checkpoint(tmp_path, layers=1, quant=quant)
    with pytest.raises(ValueError, match=match):
        ck.read_quant_config(tmp_path)


def test_quant_config_alternate_file(tmp_path: Path) -> None:
    write_checkpoint(tmp_path, layers=1, quant=None)
    assert ck.read_quant_config(tmp_path) is None
    (tmp_path / "quant_config.json").write_text(json.dumps({"w_bit": 4, "q_group_size": 64, "zero_point": True, "version": "GEMM"}))
    assert ck.read_quant_config(tmp_path) == ck.QuantConfig(4, 64, True, "gemm")


@pytest.mark.parametrize("shards", [1, 3])
def test_read_fuses_along_n(tmp_path: Path, shards: int) -> None:
    tensors = write_checkpoint(tmp_path, shards=shards)
    lin = ck.read_awq_linears(tmp_path)
    assert sorted(lin) == sorted(
        f"model.layers.{li}.{n}" for li in range(2)
        for n in ("self_attn.qkv_proj", "self_attn.o_proj", "mlp.gate_up_proj", "mlp.down_proj")
    )
    qkv = lin["model.layers.1.self_attn.qkv_proj"]
    parts = [f"model.layers.1.self_attn.{p}_proj" for p in "qkv"]
    for field, dim in (("qweight", 1), ("qzeros", 1), ("scales", 1), ("bias", 0)):
        expect = torch.cat([tensors[f"{p}.{field}"] for p in parts], dim=dim)
        assert torch.equal(getattr(qkv, field), expect)
    assert (qkv.n, qkv.k) == (H + 2 * KV, H)
    gu = lin["model.layers.0.mlp.gate_up_proj"]
    assert (gu.n, gu.k) == (2 * INTER, H) and gu.bias is None
    down = lin["model.layers.0.mlp.down_proj"]
    assert torch.equal(down.qweight, tensors["model.layers.0.mlp.down_proj.qweight"])


def test_read_without_fusion_keeps_every_linear(tmp_path: Path) -> None:
    write_checkpoint(tmp_path, layers=1)
    lin = ck.read_awq_linears(tmp_path, fuse=None)
    assert sorted(lin) == sorted(f"model.layers.0.{n}" for n in LINEARS)


def test_incomplete_layer_is_named(tmp_path: Path) -> None:
    tensors = write_checkpoint(tmp_path, layers=1)
    del tensors["model.layers.0.mlp.down_proj.scales"]
    save_file(tensors, str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match=r"incomplete AWQ layer 'model.layers.0.mlp.down_proj': missing \['scales'\]"):
        ck.read_awq_linears(tmp_path)


def test_fusion_rejects_mismatched_parts(tmp_path: Path) -> None:
    tensors = write_checkpoint(tmp_path, layers=1)
    for part, t in awq_tensors(KV, 2 * H, 9, bias=True).items():  # v_proj with another K
        tensors[f"model.layers.0.self_attn.v_proj.{part}"] = t
    save_file(tensors, str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match="different K"):
        ck.read_awq_linears(tmp_path)


def test_missing_shard_and_empty_dir(tmp_path: Path) -> None:
    write_checkpoint(tmp_path / "a", layers=1, shards=2)
    (tmp_path / "a" / "model-00002-of-00002.safetensors").unlink()
    with pytest.raises(FileNotFoundError, match="missing shards"):
        ck.checkpoint_files(tmp_path / "a")
    (tmp_path / "b").mkdir()
    with pytest.raises(FileNotFoundError, match="no \\*.safetensors"):
        ck.checkpoint_files(tmp_path / "b")


def test_load_needs_a_gpu(tmp_path: Path) -> None:
    write_checkpoint(tmp_path, layers=1)
    with pytest.raises(HipUnavailableError, match="on a gfx950 GPU"):
        ck.load_awq_checkpoint(tmp_path, device=torch.device("cpu"))
