"""Kernel-path counters with the reference's metric names and labels (metrics.py:1-76).

* ``tokenforge_kernel_calls_total{kernel,bucket}``: dispatch decisions, which shows the HIP
  kernels are the ones running;
* ``tokenforge_fallback_total{reason}``: layers the kernels cannot serve (this build has no
  per-call fallback: an op that cannot run on the GPU raises).

Counts are kept in-process per label tuple and, when ``prometheus_client`` is importable,
mirrored into a Prometheus counter family of the same name. The C++ operators count their
GPU dispatches natively; those counts are added whenever a counter is read. Only host code
counts: under HIP-graph replay the host does not run, so a captured call is counted once, at
capture.
"""

from __future__ import annotations

import threading
from collections import Counter
from collections.abc import Callable, Mapping
from typing import Any


def _prometheus_family(name: str, help_text: str, labels: tuple[str, ...]) -> Any:
    """The Prometheus counter family ``name``, registering it on first use; None without the
    client library. A second import of this module finds the family already registered."""
    try:
        import prometheus_client
    except ImportError:
        return None
    registry = prometheus_client.REGISTRY
    existing = getattr(registry, "_names_to_collectors", {}).get(name)
    if existing is not None:
        return existing
    return prometheus_client.Counter(name, help_text, list(labels))


class LabeledCounter:
    """A monotonic counter family keyed by a fixed set of label names."""

    def __init__(self, name: str, documentation: str, labelnames: tuple[str, ...]) -> None:
        self.name = name
        self.labelnames = tuple(labelnames)
        self._counts: Counter[tuple[str, ...]] = Counter()
        self._guard = threading.Lock()
        self._family = _prometheus_family(name, documentation, self.labelnames)
        self._pre_read: Callable[[], None] | None = None

    def set_pre_read(self, hook: Callable[[], None]) -> None:
        """Run ``hook`` before every read and reset: it adds counts kept elsewhere (the C++
        operators count their dispatches natively) through :meth:`inc`."""
        self._pre_read = hook

    def _fold(self) -> None:
        if self._pre_read is not None:
            self._pre_read()

    def _labels(self, given: Mapping[str, object]) -> tuple[str, ...]:
        missing = [k for k in self.labelnames if k not in given]
        extra = sorted(set(given) - set(self.labelnames))
        if missing or extra:
            raise ValueError(
                f"{self.name} takes labels {self.labelnames}; missing {missing}, unexpected {extra}"
            )
        return tuple(str(given[k]) for k in self.labelnames)

    def inc(self, amount: float = 1.0, **labels: str) -> None:
        key = self._labels(labels)
        with self._guard:
            self._counts[key] += amount
        if self._family is not None:
            self._family.labels(*key).inc(amount)

    def value(self, **labels: str) -> float:
        key = self._labels(labels)
        self._fold()
        with self._guard:
            return float(self._counts[key])

    def total(self) -> float:
        self._fold()
        with self._guard:
            return float(sum(self._counts.values()))

    def snapshot(self) -> dict[tuple[str, ...], float]:
        self._fold()
        with self._guard:
            return {key: float(v) for key, v in self._counts.items()}

    def reset(self) -> None:
        """Forget the in-process counts (tests); the Prometheus family stays monotonic."""
        self._fold()
        with self._guard:
            self._counts = Counter()


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
