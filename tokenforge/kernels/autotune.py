"""Persistent autotune cache for the gfx950 W4A16 kernels (autotune.py:1-267 in the reference).

Tuning runs eagerly at weight-load time (``process_weights_after_loading``), before HIP
graphs are captured. The hot path only does a dict lookup and falls back to the heuristic
:func:`config.default_config` on a miss, so a call never benchmarks, allocates for tuning, or
synchronizes.

Lookups fall back to a table shipped in ``tokenforge/kernels/tuned/`` (same format, tuned on
MI355X for the Qwen2.5-7B decoder shapes) and then to the heuristic default.

The cache lives at ``$TOKENFORGE_CACHE_DIR`` (default ``~/.cache/tokenforge``) as
``<gpu>-hip<abi>.json``: ``<gpu>`` is ``device.gpu_identity`` (e.g. ``amd-gfx950-256cu``)
and ``<abi>`` the kernel library's ABI version, so a rebuilt
library with different variants never reuses stale entries. Entries are keyed
``"{bucket}:{n}:{k}:{group}"`` by M bucket. Writes are atomic (tmp -> fsync -> rename ->
fsync dir). Anything unexpected on read (bad JSON, wrong schema, another GPU or ABI, an
invalid config, a config of the wrong kernel family for its bucket) discards the whole file
with a warning. A cache is never partially trusted.

Timing (the reference benchmarks each candidate with a cache flush before the call): a
candidate is launched once per copy of the layer's synthetic weights from one HIP graph, the
copies together larger than twice the 256 MB Infinity Cache, so every launch streams its
weights from HBM as consecutive decode layers do and host launch overhead is not measured.
Every candidate's output is first checked against the default config's.

Selection is two-stage. The screen times every candidate once (best of three replays), and
with over a hundred candidates the minimum of such single samples favours a config that was
merely lucky: on MI355X a screen winner ran 8% slower than the runner-up in steady state.
The best few of the screen are therefore re-timed in interleaved rounds (the order rotates
every round, so drift of the clock or of the memory system hits all of them alike) and the
lowest median wins.
"""

from __future__ import annotations

import functools
import json
import logging
import os
import statistics
import tempfile
import threading
from collections.abc import Callable, Iterable
from pathlib import Path
from typing import Any, Final

import torch

from tokenforge.kernels import _lib
from tokenforge.kernels.config import (
    M_BUCKETS,
    NUM_CUS,
    GemmConfig,
    candidate_configs,
    default_config,
    fill_split_candidates,
)

log = logging.getLogger(__name__)

SCHEMA_VERSION: Final = 1
CACHE_DIR_ENV: Final = "TOKENFORGE_CACHE_DIR"


def hip_abi() -> str:
    return str(_lib.ABI_VERSION)


def cache_dir() -> Path:
    env = os.environ.get(CACHE_DIR_ENV)
    return Path(env) if env else Path.home() / ".cache" / "tokenforge"


def cache_path(gpu: str, abi: str) -> Path:
    return cache_dir() / f"{gpu}-hip{abi}.json"


def entry_key(bucket: int, n: int, k: int, group_size: int) -> str:
    return f"{bucket}:{n}:{k}:{group_size}"


class CacheRejectedError(ValueError):
    """The on-disk cache failed validation."""


def _decode_key(key: object) -> tuple[int, int, int, int]:
    """``"{bucket}:{n}:{k}:{group}"`` -> its four integers, or CacheRejectedError."""
    fields = key.split(":") if isinstance(key, str) else ()
    if len(fields) != 4 or not all(f.isdigit() for f in fields):
        raise CacheRejectedError(f"malformed key {key!r}")
    bucket, n, k, group = map(int, fields)
    if bucket not in M_BUCKETS or min(n, k, group) <= 0 or k % group:
        raise CacheRejectedError(f"impossible key {key!r}")
    return bucket, n, k, group


def _decode_config(key: str, bucket: int, group: int, raw: object) -> GemmConfig:
    try:
        cfg = GemmConfig.from_dict(raw)
        cfg.validate(group)
    except (TypeError, ValueError) as exc:
        raise CacheRejectedError(f"invalid config for {key!r}: {exc}") from exc
    if not cfg.fits_bucket(bucket):
        raise CacheRejectedError(f"{cfg.kernel} block_m={cfg.block_m} does not fit bucket {bucket}")
    return cfg


def _decode_document(text: str, gpu: str, abi: str) -> dict[str, GemmConfig]:
    """Parse and check a whole cache file; any problem rejects all of it."""
    try:
        doc = json.loads(text)
    except json.JSONDecodeError as exc:
        raise CacheRejectedError(f"not JSON: {exc}") from exc
    if not isinstance(doc, dict):
        raise CacheRejectedError("top level is not an object")
    header = (("schema", SCHEMA_VERSION, "schema"), ("gpu", gpu, "gpu"), ("hip", abi, "kernel ABI"))
    for field, expected, what in header:
        if doc.get(field) != expected:
            raise CacheRejectedError(f"{what} {doc.get(field)!r} != {expected!r} of this process")
    raw = doc.get("entries")
    if not isinstance(raw, dict):
        raise CacheRejectedError("'entries' is not an object")
    table: dict[str, GemmConfig] = {}
    for key, value in raw.items():
        bucket, _n, _k, group = _decode_key(key)
        table[key] = _decode_config(key, bucket, group, value)
    return table


def _encode_document(gpu: str, abi: str, table: dict[str, GemmConfig]) -> str:
    doc = {
        "schema": SCHEMA_VERSION,
        "gpu": gpu,
        "hip": abi,
        "torch": torch.__version__,
        "entries": {key: table[key].to_dict() for key in sorted(table)},
    }
    return json.dumps(doc, indent=1, sort_keys=True) + "\n"


def _replace_file(path: Path, text: str) -> None:
    """Write ``text`` to ``path`` so a reader sees the old file or the whole new one: a
    temporary file in the same directory is synced, renamed over ``path``, and the directory
    entry is synced. A failure removes the temporary file and leaves ``path`` untouched."""
    path.parent.mkdir(parents=True, exist_ok=True)
    with tempfile.NamedTemporaryFile(
        "w", encoding="utf-8", dir=path.parent, prefix=f".{path.name}.", suffix=".tmp", delete=False
    ) as tmp:
        staged = Path(tmp.name)
        try:
            tmp.write(text)
            tmp.flush()
            os.fsync(tmp.fileno())
        except BaseException:
            staged.unlink(missing_ok=True)
            raise
    try:
        os.replace(staged, path)
    except BaseException:
        staged.unlink(missing_ok=True)
        raise
    dir_fd = os.open(path.parent, os.O_RDONLY)
    try:
        os.fsync(dir_fd)
    finally:
        os.close(dir_fd)


class AutotuneCache:
    """The tuned configs of one (GPU, kernel ABI) pair, backed by one JSON file."""

    def __init__(self, path: Path, gpu: str, abi: str) -> None:
        self.path = path
        self.gpu = gpu
        self.abi = abi
        self.discarded_reason: str | None = None
        self._table: dict[str, GemmConfig] = {}
        self._mutex = threading.Lock()

    def load(self) -> None:
        """Read the file: a missing file is an empty cache, an invalid one is discarded whole."""
        self.discarded_reason = None
        try:
            table = _decode_document(self.path.read_text(encoding="utf-8"), self.gpu, self.abi)
        except FileNotFoundError:
            table = {}
        except (OSError, UnicodeDecodeError) as exc:
            self._reject(f"unreadable: {exc}")
            return
        except CacheRejectedError as exc:
            self._reject(str(exc))
            return
        with self._mutex:
            self._table = table
        _changed()

    def _reject(self, reason: str) -> None:
        log.warning("autotune cache %s discarded (%s); configs will be retuned", self.path, reason)
        self.discarded_reason = reason
        with self._mutex:
            self._table = {}
        _changed()

    def get(self, bucket: int, n: int, k: int, group_size: int) -> GemmConfig | None:
        return self._table.get(entry_key(bucket, n, k, group_size))

    def put(self, bucket: int, n: int, k: int, group_size: int, cfg: GemmConfig) -> None:
        cfg.validate(group_size)
        if not cfg.fits_bucket(bucket):
            raise ValueError(f"{cfg} does not fit bucket {bucket}")
        with self._mutex:
            self._table = {**self._table, entry_key(bucket, n, k, group_size): cfg}
        _changed()

    def __len__(self) -> int:
        return len(self._table)

    def save(self) -> None:
        with self._mutex:
            text = _encode_document(self.gpu, self.abi, self._table)
        _replace_file(self.path, text)


_REGISTRY: dict[tuple[str, str], AutotuneCache] = {}
_REGISTRY_MUTEX = threading.Lock()
_CHANGE_HOOKS: list[Callable[[], None]] = []


def on_change(hook: Callable[[], None]) -> None:
    """Call ``hook`` whenever a config :func:`lookup` returns may change (a cache loaded, put,
    discarded or reset): holders of launch decisions made from lookups drop them."""
    _CHANGE_HOOKS.append(hook)


def _changed() -> None:
    for hook in _CHANGE_HOOKS:
        hook()


def get_cache(gpu: str) -> AutotuneCache:
    """The process-wide cache of ``gpu`` for the loaded kernel ABI, read from disk once."""
    key = (gpu, hip_abi())
    with _REGISTRY_MUTEX:
        if key not in _REGISTRY:
            cache = AutotuneCache(cache_path(*key), *key)
            cache.load()
            _REGISTRY[key] = cache
        return _REGISTRY[key]


def reset_caches() -> None:
    with _REGISTRY_MUTEX:
        _REGISTRY.clear()
    _changed()


SHIPPED_DIR: Final = Path(__file__).resolve().parent / "tuned"
"""Tuned tables shipped with the package, one file per (GPU, kernel ABI) in the cache format."""


@functools.cache
def shipped_table(gpu: str, abi: str) -> dict[str, GemmConfig]:
    """The shipped table for this GPU and kernel ABI (empty when there is none). It is read with
    the cache's own strict decoder: a file that fails any check is not used at all."""
    path = SHIPPED_DIR / cache_path(gpu, abi).name
    try:
        return _decode_document(path.read_text(encoding="utf-8"), gpu, abi)
    except FileNotFoundError:
        return {}
    except (OSError, UnicodeDecodeError, CacheRejectedError) as exc:
        log.warning("shipped autotune table %s ignored (%s)", path, exc)
        return {}


def config_source(gpu: str, bucket: int, n: int, k: int, group_size: int) -> str:
    """Where :func:`lookup` takes this entry from: "cache", "shipped" or "default"."""
    if get_cache(gpu).get(bucket, n, k, group_size) is not None:
        return "cache"
    if entry_key(bucket, n, k, group_size) in shipped_table(gpu, hip_abi()):
        return "shipped"
    return "default"


def lookup(gpu: str, bucket: int, n: int, k: int, group_size: int) -> GemmConfig:
    """Hot-path lookup: the config tuned on this machine if cached, else the table shipped for
    this GPU and kernel ABI, else the heuristic default."""
    tuned = get_cache(gpu).get(bucket, n, k, group_size)
    if tuned is not None:
        return tuned
    shipped = shipped_table(gpu, hip_abi()).get(entry_key(bucket, n, k, group_size))
    return default_config(bucket, n, k, group_size) if shipped is None else shipped


BenchFn = Callable[[Callable[[], object]], float]

_FLUSH_BYTES = 512 * 1024 * 1024
"""Larger than MI355X's 256 MB Infinity Cache, so each timed call reads weights from HBM."""


@functools.cache
def _flush_buffer(index: int) -> torch.Tensor:
    return torch.empty(_FLUSH_BYTES // 4, dtype=torch.int32, device=torch.device("cuda", index))


def hip_bench(fn: Callable[[], object], warmup: int = 5, rep: int = 25) -> float:
    """Median runtime of ``fn`` in ms, device caches flushed before every timed call."""
    flush = _flush_buffer(torch.cuda.current_device())
    for _ in range(warmup):
        fn()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(rep)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(rep)]
    for s, e in zip(starts, ends):
        flush.zero_()
        s.record()
        fn()
        e.record()
    torch.cuda.synchronize()
    return float(statistics.median(s.elapsed_time(e) for s, e in zip(starts, ends)))


_COLD_BYTES = 640 * 1024 * 1024
"""Weight bytes the default tuner rotates through: more than twice the 256 MB Infinity Cache."""
_MAX_COPIES = 64


def graph_bench(fns: list[Callable[[], object]], reps: int = 3) -> float:
    """Per-launch time in ms of one HIP-graph replay launching each of ``fns`` once, best of
    ``reps`` replays. The graph removes host launch overhead; ``fns`` rotate over distinct
    weight copies so each launch reads its weights from HBM, as consecutive decode layers do."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        for f in fns[:2]:
            f()
        stream.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            for f in fns:
                f()
    torch.cuda.current_stream().wait_stream(stream)
    graph.replay()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        end.record()
        torch.cuda.synchronize()
        best = min(best, start.elapsed_time(end) / len(fns))
    return best


FINALISTS: Final = 6
"""Screen winners re-timed by :func:`select_finalist`."""
FINAL_ROUNDS: Final = 5


def select_finalist(
    screened: list[tuple[float, GemmConfig]],
    time_cfg: Callable[[GemmConfig], float],
    finalists: int = FINALISTS,
    rounds: int = FINAL_ROUNDS,
) -> GemmConfig:
    """The config with the lowest median over ``rounds`` interleaved re-timings among the
    ``finalists`` fastest of ``screened`` (``(time, config)`` pairs); ties go to the better
    screen time. Round r times the finalists starting from the r-th, so no config is always
    first or last."""
    ranked = sorted(screened, key=lambda r: r[0])[:finalists]
    if not ranked:
        raise ValueError("no screened candidates")
    if len(ranked) == 1:
        return ranked[0][1]
    samples: list[list[float]] = [[] for _ in ranked]
    n = len(ranked)
    for r in range(rounds):
        for j in range(n):
            i = (r + j) % n
            samples[i].append(time_cfg(ranked[i][1]))
    best = min(range(n), key=lambda i: (statistics.median(samples[i]), ranked[i][0]))
    return ranked[best][1]


def synthetic_layer(
    n: int, k: int, group_size: int, device: torch.device, seed: int = 0
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Random AWQ-distributed layer in the tile layout the kernels read: nibbles and
    zero-points uniform in [0, 15], fp16 scales uniform in [1e-3, 1e-2]. Returns
    ``(qweight_t, scales, qzeros)``."""
    from tokenforge.kernels.hip.layout import tile_pack
    from tokenforge.kernels.pack import pack_int4

    gen = torch.Generator(device=device).manual_seed(seed)
    q = torch.randint(0, 16, (n, k), generator=gen, device=device, dtype=torch.int32)
    z = torch.randint(0, 16, (k // group_size, n), generator=gen, device=device, dtype=torch.int32)
    s = (torch.rand((k // group_size, n), generator=gen, device=device) * 9e-3 + 1e-3).to(torch.float16)
    return tile_pack(pack_int4(q), s, pack_int4(z), group_size)


def tune_layer(
    n: int,
    k: int,
    group_size: int,
    *,
    device: torch.device,
    gpu: str,
    buckets: Iterable[int] = M_BUCKETS,
    bench_fn: BenchFn | None = None,
    candidates: Callable[[int, int], list[GemmConfig]] = candidate_configs,
    save: bool = True,
) -> dict[int, GemmConfig]:
    """Tune every M bucket for one (N, K) layer shape and persist the winners.

    Each candidate is checked against the default config's output before it can win, so a
    config that miscomputes is never cached. Buckets already in the cache are skipped, and
    nothing touches the device when every bucket is cached.
    """
    from tokenforge.kernels.hip.w4a16 import w4a16_gemm

    cache = get_cache(gpu)
    buckets = list(buckets)
    winners: dict[int, GemmConfig] = {}
    todo = []
    for bucket in buckets:
        cached = cache.get(bucket, n, k, group_size)
        if cached is not None:
            winners[bucket] = cached
        else:
            todo.append(bucket)
    if not todo:
        return winners
    rotating = bench_fn is None
    if rotating and device.type != "cuda":
        raise RuntimeError("tuning needs a CUDA (HIP) device or an explicit bench_fn")

    # Default timing: a HIP graph over `copies` distinct weight copies (see graph_bench).
    copies = 1
    if rotating:
        copies = max(2, min(_MAX_COPIES, -(-_COLD_BYTES // max(1, n * k // 2))))
    layers = [synthetic_layer(n, k, group_size, device, seed=i) for i in range(copies)]
    qweight_t, scales, qzeros = layers[0]
    gen = torch.Generator(device=device).manual_seed(1)
    for bucket in todo:
        x = (torch.randn((bucket, k), generator=gen, device=device) * 0.5).to(torch.float16)
        base_cfg = default_config(bucket, n, k, group_size)
        ref = w4a16_gemm(x, qweight_t, scales, qzeros, group_size, base_cfg).float()
        tol = 1e-2 * float(ref.abs().max()) + 1e-3
        screened: list[tuple[float, GemmConfig]] = []
        cands = candidates(bucket, group_size)
        cands = cands + fill_split_candidates(cands, bucket, n, k, NUM_CUS)
        for cfg in cands:
            try:
                out = w4a16_gemm(x, qweight_t, scales, qzeros, group_size, cfg)
                if float((out.float() - ref).abs().max()) > tol:
                    log.warning("config %s miscomputes for %s; skipped", cfg, (bucket, n, k))
                    continue
                if rotating:
                    t = graph_bench(
                        [functools.partial(w4a16_gemm, x, *lay, group_size, cfg) for lay in layers]
                    )
                else:
                    assert bench_fn is not None
                    t = bench_fn(
                        functools.partial(w4a16_gemm, x, qweight_t, scales, qzeros, group_size, cfg)
                    )
            except (ValueError, RuntimeError) as exc:  # variant cannot run this shape
                log.debug("config %s failed to run: %s", cfg, exc)
                continue
            screened.append((t, cfg))
        if not screened:
            chosen = base_cfg
        elif rotating:
            chosen = select_finalist(
                screened,
                lambda cfg: graph_bench(
                    [functools.partial(w4a16_gemm, x, *lay, group_size, cfg) for lay in layers]
                ),
            )
        else:  # an explicit bench_fn is trusted as given: the screen decides
            chosen = min(screened, key=lambda r: r[0])[1]
        cache.put(bucket, n, k, group_size, chosen)
        winners[bucket] = chosen
    del layers
    if save:
        cache.save()
    return winners
