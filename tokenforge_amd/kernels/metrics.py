"""Kernel-path counters (metrics.py:1-76 in the reference).

``tokenforge_kernel_calls_total{kernel,bucket}`` proves the HIP path is running and
``tokenforge_fallback_total{reason}`` counts layers that cannot be served (this build has no
per-call fallback: an op that cannot run on the GPU raises). Counters are host-side and
count dispatch decisions; under HIP-graph replay the host code does not run, so captured
calls are counted once, at capture. When ``prometheus_client`` is importable the counters
are exported through it as well.
"""

from __future__ import annotations

import threading
from collections import defaultdict
from typing import Any


class LabeledCounter:
    def __init__(self, name: str, documentation: str, labelnames: tuple[str, ...]) -> None:
        self.name = name
        self.labelnames = labelnames
        self._values: defaultdict[tuple[str, ...], float] = defaultdict(float)
        self._lock = threading.Lock()
        self._prom: Any = None
        try:
            import prometheus_client
        except ImportError:
            return
        try:
            self._prom = prometheus_client.Counter(name, documentation, labelnames)
        except ValueError:  # already registered (module imported twice)
            self._prom = prometheus_client.REGISTRY._names_to_collectors.get(name)

    def _key(self, labels: dict[str, str]) -> tuple[str, ...]:
        if set(labels) != set(self.labelnames):
            raise ValueError(f"{self.name} expects labels {self.labelnames}, got {sorted(labels)}")
        return tuple(str(labels[k]) for k in self.labelnames)

    def inc(self, amount: float = 1.0, **labels: str) -> None:
        key = self._key(labels)
        with self._lock:
            self._values[key] += amount
        if self._prom is not None:
            self._prom.labels(*key).inc(amount)

    def value(self, **labels: str) -> float:
        with self._lock:
            return self._values.get(self._key(labels), 0.0)

    def total(self) -> float:
        with self._lock:
            return sum(self._values.values())

    def snapshot(self) -> dict[tuple[str, ...], float]:
        with self._lock:
            return dict(self._values)

    def reset(self) -> None:
        """Clear the in-process view (tests only; Prometheus counters are monotonic)."""
        with self._lock:
            self._values.clear()


KERNEL_CALLS = LabeledCounter(
    "tokenforge_kernel_calls",
    "TokenForge kernel dispatches by kernel and M bucket",
    ("kernel", "bucket"),
)
FALLBACKS = LabeledCounter(
    "tokenforge_fallback",
    "TokenForge layers not served by the HIP kernels, by reason",
    ("reason",),
)
