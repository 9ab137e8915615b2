"""bench.py's bookkeeping (micro.py:133-181, env.py:51-85 in the reference), on CPU: the
regression gate against a committed baseline, the baseline update, and the fingerprint's
code-tree hash."""

from __future__ import annotations

import json
from pathlib import Path

import pytest

import bench


def _line(value: float = 100.0, scale: float = 1.0) -> dict:  # type: ignore[type-arg]
    return {
        "gpu": "amd-gfx950-256cu",
        "value": value,
        "per_shape": [{"layer": "o_proj", "m": 1, "us": 4.0 * scale}, {"layer": "down_proj", "m": 1, "us": 11.0}],
        "gemm_small_m": [{"layer": "gate_up_proj", "m": 16, "us": 27.0}],
        "gemm_w4a8_fp8": [{"layer": "down_proj", "m": 256, "us": 46.0}],
        "rmsnorm_fp8": [{"t": 4096, "us": 11.0}],
        "vendor_fp16": [{"layer": "o_proj", "m": 1, "us": 9.0}],
        "stack": [{"m": 1, "fused": {"ms_per_pass": 1.4}}],
        "env": {"code_tree": "abc", "git_sha": None},
    }


def test_timed_rows_keys() -> None:
    rows = bench.timed_rows(_line())
    assert rows == {"hip|o_proj|1": 4.0, "hip|down_proj|1": 11.0, "hip-cfg4|gate_up_proj|16": 27.0,
                    "hip-fp8|down_proj|256": 46.0, "hip|rmsnorm_fp8|4096": 11.0, "vendor-fp16|o_proj|1": 9.0,
                    "hip-stack|fused|1": pytest.approx(1400.0)}


def test_regression_gate_flags_entries_more_than_five_percent_slower(tmp_path: Path) -> None:
    path = tmp_path / "baseline.json"
    assert bench.regression_check(_line(), path) is None  # no committed baseline: no gate
    bench.update_baseline(_line(), "first", path)
    doc = json.loads(path.read_text())
    assert doc["amd-gfx950-256cu"]["reason"] == "first" and doc["amd-gfx950-256cu"]["value"] == 100.0
    same = bench.regression_check(_line(), path)
    assert same is not None and same["pass"] and same["compared"] == 7 and same["value_vs_baseline"] == 1.0
    within = bench.regression_check(_line(scale=1.049), path)
    assert within is not None and within["pass"]
    slower = bench.regression_check(_line(value=90.0, scale=1.06), path)
    assert slower is not None and not slower["pass"]
    assert [r["entry"] for r in slower["regressions"]] == ["hip|o_proj|1"]
    assert slower["value_vs_baseline"] == pytest.approx(0.9)
    other = dict(_line(), gpu="some-other-gpu")
    assert bench.regression_check(other, path)["compared"] == 0  # type: ignore[index]


def test_code_tree_hash_is_stable_and_covers_the_sources() -> None:
    h = bench.code_tree_hash()
    assert len(h) == 64 and h == bench.code_tree_hash()
    assert all((bench.ROOT / p).exists() for p in bench.CODE_PATHS)
