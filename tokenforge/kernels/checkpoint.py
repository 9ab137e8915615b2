"""Load-time pipeline for a local AWQ checkpoint: read, validate, GPU repack, autotune.

The reference consumes the AWQ GEMM format unchanged (docs/adr/0002-consume-awq-format.md)
and plans this flow for its vLLM plugin's ``process_weights_after_loading`` ("repack once",
then tune; README.md:67-69, autotune.py:1-10). This module is that flow for a checkpoint on
local disk, without vLLM:

1. :func:`read_quant_config` reads the AWQ settings of the checkpoint directory
   (``config.json``'s ``quantization_config``, or ``quant_config.json`` /
   ``quantize_config.json``) and rejects anything but 4-bit, zero-point, GEMM-version AWQ.
2. :func:`read_awq_linears` reads the safetensors file(s) on the host (one file, a directory
   of shards, or shards named by ``model.safetensors.index.json``) and groups the tensors of
   every AWQ linear by name prefix: ``<prefix>.qweight`` int32 ``[K, N/8]``,
   ``<prefix>.qzeros`` int32 ``[K/G, N/8]``, ``<prefix>.scales`` fp16 ``[K/G, N]`` and an
   optional ``<prefix>.bias``. Linears a serving engine runs as one GEMM (Qwen2: q/k/v and
   gate/up) are concatenated along N before the repack; AWQ packs along N in groups of 8,
   so concatenating the packed tensors is exact.
3. :func:`load_awq_checkpoint` checks each linear against the HIP path
   (``dispatch.layer_support``; unsupported ones are reported, counted in
   ``tokenforge_fallback_total`` and left to the caller), validates and repacks the supported
   ones on the GPU (``pack.pack_awq``), then tunes every distinct (N, K) shape into the
   autotune cache file (``autotune.tune_layer``).

Step 3 runs on a gfx950 GPU (the layer support check and the tuning need one) and raises for
a non-GPU device.
"""

from __future__ import annotations

import json
from dataclasses import dataclass, field
from pathlib import Path
from typing import Iterable, Mapping

import torch

from tokenforge.kernels import autotune, dispatch
from tokenforge.kernels.config import M_BUCKETS
from tokenforge.kernels.pack import PACK_FACTOR, W4A16Weights, pack_awq

AWQ_PARTS = ("qweight", "qzeros", "scales")
QWEN2_FUSIONS: Mapping[str, tuple[str, ...]] = {
    "qkv_proj": ("q_proj", "k_proj", "v_proj"),
    "gate_up_proj": ("gate_proj", "up_proj"),
}
"""Fused linear name -> the checkpoint linears it concatenates along N, in order."""
INDEX_FILE = "model.safetensors.index.json"
_QUANT_CONFIG_FILES = ("quant_config.json", "quantize_config.json")


@dataclass(frozen=True)
class QuantConfig:
    bits: int
    group_size: int
    zero_point: bool
    version: str


@dataclass(frozen=True)
class AwqLinear:
    """One linear in AWQ GEMM format (host tensors, as stored)."""

    qweight: torch.Tensor
    qzeros: torch.Tensor
    scales: torch.Tensor
    bias: torch.Tensor | None

    @property
    def k(self) -> int:
        return int(self.qweight.shape[0])

    @property
    def n(self) -> int:
        return int(self.qweight.shape[1]) * PACK_FACTOR


@dataclass
class LoadedCheckpoint:
    group_size: int
    layers: dict[str, tuple[W4A16Weights, torch.Tensor | None]] = field(default_factory=dict)
    fallbacks: dict[str, str] = field(default_factory=dict)
    tuned: dict[tuple[int, int], dict[int, object]] = field(default_factory=dict)


def _parse_quant(q: Mapping[str, object], source: str) -> QuantConfig:
    method = str(q.get("quant_method", "awq")).lower()
    if method != "awq":
        raise ValueError(f"{source}: quant_method {method!r} is not AWQ")
    bits = int(q.get("bits", q.get("w_bit", 4)))  # type: ignore[arg-type]
    group = int(q.get("group_size", q.get("q_group_size", 128)))  # type: ignore[arg-type]
    zero_point = bool(q.get("zero_point", True))
    version = str(q.get("version", "gemm")).lower()
    if bits != 4:
        raise ValueError(f"{source}: {bits}-bit AWQ is not supported (4-bit only)")
    if not zero_point:
        raise ValueError(f"{source}: AWQ without zero points is not supported")
    if version != "gemm":
        raise ValueError(f"{source}: AWQ version {version!r} is not the GEMM layout")
    return QuantConfig(bits, group, zero_point, version)


def read_quant_config(path: str | Path) -> QuantConfig | None:
    """AWQ settings of a checkpoint directory (or of a file's directory); None if absent."""
    d = Path(path)
    if d.is_file():
        d = d.parent
    cfg = d / "config.json"
    if cfg.is_file():
        q = json.loads(cfg.read_text()).get("quantization_config")
        if q is not None:
            return _parse_quant(q, str(cfg))
    for name in _QUANT_CONFIG_FILES:
        f = d / name
        if f.is_file():
            return _parse_quant(json.loads(f.read_text()), str(f))
    return None


def checkpoint_files(path: str | Path) -> list[Path]:
    """The safetensors files of a checkpoint: the file itself, the shards its index names, or
    every ``*.safetensors`` of the directory."""
    p = Path(path)
    if p.is_file():
        return [p]
    if not p.is_dir():
        raise FileNotFoundError(f"no checkpoint at {p}")
    index = p / INDEX_FILE
    if index.is_file():
        names = sorted(set(json.loads(index.read_text())["weight_map"].values()))
        files = [p / n for n in names]
        missing = [str(f) for f in files if not f.is_file()]
        if missing:
            raise FileNotFoundError(f"{index} names missing shards: {missing}")
        return files
    files = sorted(p.glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"no *.safetensors in {p}")
    return files


def _concat(parts: list[AwqLinear], name: str) -> AwqLinear:
    k = parts[0].k
    if any(p.k != k for p in parts):
        raise ValueError(f"cannot fuse {name}: its parts have different K ({[p.k for p in parts]})")
    if any(p.qzeros.shape[0] != parts[0].qzeros.shape[0] for p in parts):
        raise ValueError(f"cannot fuse {name}: its parts have different group counts")
    has_bias = [p.bias is not None for p in parts]
    if any(has_bias) and not all(has_bias):
        raise ValueError(f"cannot fuse {name}: only some of its parts have a bias")
    return AwqLinear(
        qweight=torch.cat([p.qweight for p in parts], dim=1),
        qzeros=torch.cat([p.qzeros for p in parts], dim=1),
        scales=torch.cat([p.scales for p in parts], dim=1),
        bias=torch.cat([p.bias for p in parts]) if all(has_bias) else None,  # type: ignore[misc]
    )


def read_awq_linears(
    path: str | Path, *, fuse: Mapping[str, Iterable[str]] | None = QWEN2_FUSIONS
) -> dict[str, AwqLinear]:
    """Every AWQ linear of the checkpoint, by name prefix, on the host; fused per ``fuse``."""
    from safetensors import safe_open

    found: dict[str, dict[str, torch.Tensor]] = {}
    for f in checkpoint_files(path):
        with safe_open(str(f), framework="pt", device="cpu") as st:
            for key in st.keys():
                prefix, _, part = key.rpartition(".")
                if part in AWQ_PARTS or part == "bias":
                    found.setdefault(prefix, {})[part] = st.get_tensor(key)
    linears: dict[str, AwqLinear] = {}
    for prefix, parts in sorted(found.items()):
        if not any(p in parts for p in AWQ_PARTS):
            continue  # a bias of a layer that is not quantized
        missing = [p for p in AWQ_PARTS if p not in parts]
        if missing:
            raise ValueError(f"incomplete AWQ layer {prefix!r}: missing {missing}")
        linears[prefix] = AwqLinear(parts["qweight"], parts["qzeros"], parts["scales"], parts.get("bias"))
    for fused, members in (fuse or {}).items():
        members = tuple(members)
        heads = [p for p in linears if p.rsplit(".", 1)[-1] == members[0]]
        for head in heads:
            parent = head.rsplit(".", 1)[0] if "." in head else ""
            names = [f"{parent}.{m}" if parent else m for m in members]
            if not all(n in linears for n in names):
                continue
            linears[f"{parent}.{fused}" if parent else fused] = _concat([linears.pop(n) for n in names], fused)
    return dict(sorted(linears.items()))


def load_awq_checkpoint(
    path: str | Path,
    *,
    device: torch.device,
    group_size: int | None = None,
    tune_buckets: Iterable[int] | None = M_BUCKETS,
    gpu: str | None = None,
    backend: dispatch.Backend | None = None,
    fuse: Mapping[str, Iterable[str]] | None = QWEN2_FUSIONS,
) -> LoadedCheckpoint:
    """Read, validate, repack on the GPU and tune (``tune_buckets``; None or empty skips tuning)."""
    from tokenforge.kernels.device import device_arch, gpu_identity

    if device.type != "cuda":
        raise dispatch.HipUnavailableError(
            f"AWQ checkpoints are repacked and tuned on a gfx950 GPU; got device {device}"
        )
    cfg = read_quant_config(path)
    if cfg is not None and group_size is not None and group_size != cfg.group_size:
        raise ValueError(f"group_size {group_size} disagrees with the checkpoint's {cfg.group_size}")
    g = group_size if group_size is not None else (cfg.group_size if cfg is not None else None)
    if g is None:
        raise ValueError("the checkpoint has no AWQ config; pass group_size")
    backend = backend if backend is not None else dispatch.backend_from_env()
    arch = device_arch(device)
    out = LoadedCheckpoint(group_size=g)
    for name, lin in read_awq_linears(path, fuse=fuse).items():
        reason = dispatch.layer_support(lin.n, lin.k, g, str(lin.scales.dtype).replace("torch.", ""), arch, backend)
        if reason is not None:
            dispatch.record_layer_fallback(reason)
            out.fallbacks[name] = reason
            continue
        w = pack_awq(lin.qweight.to(device), lin.qzeros.to(device), lin.scales.to(device), g)
        bias = lin.bias.to(device=device, dtype=torch.float16) if lin.bias is not None else None
        out.layers[name] = (w, bias)
    buckets = tuple(tune_buckets or ())
    if buckets:
        ident = gpu if gpu is not None else gpu_identity(device)
        for n, k in sorted({(w.n, w.k) for w, _ in out.layers.values()}):
            out.tuned[(n, k)] = autotune.tune_layer(n, k, g, device=device, gpu=ident, buckets=buckets)  # type: ignore[assignment]
    return out
