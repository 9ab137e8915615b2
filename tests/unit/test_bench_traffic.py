"""bench.py's HBM-traffic bookkeeping: ``--traffic-summary`` turns two counter runs of
``--traffic-probe`` into the committed summary, and ``committed_traffic`` finds the row of the
config in use. Synthetic counter files with known values; no GPU."""

from __future__ import annotations

import csv
import json
from pathlib import Path

import pytest

import bench

CFGS = [
    {"kernel": "gemv_dot", "block_m": 1, "block_n": 16, "block_k": 128, "split_k": 1, "num_warps": 4, "num_stages": 2},
    {"kernel": "gemv_mfma", "block_m": 16, "block_n": 16, "block_k": 128, "split_k": 1, "num_warps": 4, "num_stages": 4},
]
LAUNCHES = 3
CALIB = 256 << 20


def _write_run(d: Path, counter: str, gemv_kib: list[float], calib_kib: float) -> None:
    d.mkdir(parents=True)
    rows = []
    did = 1
    for v in gemv_kib:
        rows.append({"Dispatch_Id": did, "Kernel_Name": "void tf::gemv_dot_kernel<1, 1, 2, 16, true>(...)",
                     "Counter_Name": counter, "Counter_Value": v})
        did += 1
    for _ in range(4):
        rows.append({"Dispatch_Id": did, "Kernel_Name": "void at::native::neg_kernel(...)",
                     "Counter_Name": counter, "Counter_Value": calib_kib})
        did += 1
    rows.reverse()  # the summary must order by dispatch id, not by file order
    with open(d / "pmc_counter_collection.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


def test_summary_rows_and_lookup(tmp_path: Path, monkeypatch: pytest.MonkeyPatch) -> None:
    summary = tmp_path / "traffic.md"
    monkeypatch.setattr(bench, "TRAFFIC_SUMMARY", summary)
    # FETCH_SIZE counts half the bytes (scale 2), WRITE_SIZE all of them (scale 1).
    fetch = [1000.0] * LAUNCHES + [2000.0] * LAUNCHES
    write = [10.0] * LAUNCHES + [30.0] * LAUNCHES
    _write_run(tmp_path / "f", "FETCH_SIZE", fetch, CALIB / 1024 / 2)
    _write_run(tmp_path / "w", "WRITE_SIZE", write, CALIB / 1024)
    probe = {"traffic_probe": {"launches": LAUNCHES, "configs": CFGS, "algorithmic_bytes": 4096000,
                               "calibration_bytes_in": CALIB, "calibration_bytes_out": CALIB}}
    log = tmp_path / "probe.log"
    log.write_text("noise\n" + json.dumps(probe) + "\n")
    assert bench.traffic_summary(str(tmp_path / "f"), str(tmp_path / "w"), str(log)) == 0
    text = summary.read_text()
    assert "| gemv_dot bm1 bn16 bk128 w4 st2 |" in text
    assert bench.committed_traffic(CFGS[0]) == pytest.approx(1000 * 1024 * 2 + 10 * 1024)
    assert bench.committed_traffic(CFGS[1]) == pytest.approx(2000 * 1024 * 2 + 30 * 1024)
    other = dict(CFGS[0], num_warps=8)
    assert bench.committed_traffic(other) is None


def test_summary_rejects_a_dispatch_count_mismatch(tmp_path: Path, monkeypatch: pytest.MonkeyPatch) -> None:
    monkeypatch.setattr(bench, "TRAFFIC_SUMMARY", tmp_path / "traffic.md")
    _write_run(tmp_path / "f", "FETCH_SIZE", [1.0] * (LAUNCHES * 2 - 1), 1.0)
    _write_run(tmp_path / "w", "WRITE_SIZE", [1.0] * (LAUNCHES * 2), 1.0)
    log = tmp_path / "probe.log"
    log.write_text(json.dumps({"traffic_probe": {"launches": LAUNCHES, "configs": CFGS, "algorithmic_bytes": 1,
                                                 "calibration_bytes_in": CALIB}}) + "\n")
    with pytest.raises(ValueError, match="GEMV dispatches"):
        bench.traffic_summary(str(tmp_path / "f"), str(tmp_path / "w"), str(log))
    assert not (tmp_path / "traffic.md").exists()


def test_committed_summary_parses() -> None:
    """The committed summary (if any) is well formed: every machine line names a config."""
    if not bench.TRAFFIC_SUMMARY.is_file():
        pytest.skip("no committed traffic summary")
    lines = [ln for ln in bench.TRAFFIC_SUMMARY.read_text().splitlines() if ln.startswith("traffic: ")]
    assert lines
    for ln in lines:
        value, cfg = ln[len("traffic: "):].split(" ", 1)
        assert float(value) > 0
        assert bench.committed_traffic(json.loads(cfg)) == float(value)


def test_mfma_summary_from_synthetic_counters(tmp_path: Path, monkeypatch: pytest.MonkeyPatch) -> None:
    """--mfma-summary: the first `launches` GEMM dispatches per layer (in dispatch order) are the
    counted ones; busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / XCDs * SIMDs)."""
    monkeypatch.setattr(bench, "MFMA_SUMMARY", tmp_path / "mfma.md")
    d = tmp_path / "pmc"
    d.mkdir()
    rows = []
    did = 1
    cycles = 200_000.0  # per XCD
    for layer_busy in (0.30, 0.20):
        for _ in range(bench.MFMA_LAUNCHES):
            for c in bench.MFMA_COUNTERS:
                v = {"SQ_VALU_MFMA_BUSY_CYCLES": layer_busy * cycles * bench.NUM_SIMDS,
                     "GRBM_GUI_ACTIVE": cycles * bench.NUM_XCDS}.get(c, 1.0)
                rows.append({"Dispatch_Id": did, "Kernel_Name": "void tf::gemm2_kernel<256, 192, 4, 2, 3>(...)",
                             "Counter_Name": c, "Counter_Value": v})
            did += 1
    for c in bench.MFMA_COUNTERS:  # a reduce kernel and a later (graph-timing) dispatch: ignored
        rows.append({"Dispatch_Id": did, "Kernel_Name": "void tf::splitk_reduce_kernel(...)",
                     "Counter_Name": c, "Counter_Value": 5.0})
        rows.append({"Dispatch_Id": did + 1, "Kernel_Name": "void tf::gemm2_kernel<256, 192, 4, 2, 3>(...)",
                     "Counter_Name": c, "Counter_Value": 9.0})
    rows.reverse()
    with open(d / "pmc_counter_collection.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    cfg = {"kernel": "gemm_mfma", "block_m": 256, "block_n": 192, "block_k": 64, "split_k": 1, "num_warps": 8,
           "num_stages": 3}
    runs = [{"layer": "gate_up_proj", "m": 256, "n": 37888, "k": 3584, "config": cfg, "us": 100.0, "tflops": 700.0},
            {"layer": "down_proj", "m": 256, "n": 3584, "k": 18944, "config": cfg, "us": 60.0, "tflops": 580.0}]
    log = tmp_path / "probe.log"
    log.write_text(json.dumps({"mfma_probe": {"launches": bench.MFMA_LAUNCHES, "runs": runs}}) + "\n")
    assert bench.mfma_summary(str(d), str(log), str(log)) == 0
    text = (tmp_path / "mfma.md").read_text()
    assert "| gate_up_proj | gemm_mfma bm256 bn192 bk64 sk1 w8 st3 | 30.0% | 100.00 | 700.0 | 28.0% |" in text
    assert "| down_proj | gemm_mfma bm256 bn192 bk64 sk1 w8 st3 | 20.0% |" in text


def test_stats_summary_matches_dispatches_to_shapes(tmp_path: Path, monkeypatch: pytest.MonkeyPatch) -> None:
    """--stats-summary: per shape and M, the rocprofv3 rows are the dispatches of the tuned
    kernel instance with the shape's grid; different M sharing an instance split by phase."""
    monkeypatch.setattr(bench, "STATS_SUMMARY", tmp_path / "stats.md")
    d = tmp_path / "prof" / "vm"
    d.mkdir(parents=True)
    with open(d / "1_kernel_stats.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Name", "Calls", "AverageNs", "MinNs", "MaxNs", "Percentage"])
        w.writeheader()
        w.writerow({"Name": "void tf::(anonymous namespace)::gemv_dot_kernel<1, 1, 4, 8, true, true>(tf::LinearArgs, int)",
                    "Calls": 3, "AverageNs": 20000, "MinNs": 19000, "MaxNs": 21000, "Percentage": 50.0})
    dot = {"kernel": "gemv_dot", "block_m": 1, "block_n": 16, "block_k": 256, "split_k": 1, "num_warps": 4, "num_stages": 4}
    mfma = {"kernel": "gemv_mfma", "block_m": 16, "block_n": 16, "block_k": 256, "split_k": 1, "num_warps": 4,
            "num_stages": 2}
    grid = -(-(-(-37888 // 16)) // 4) * 64 * 4
    trace = []
    t = 0
    for name, dur, n in (("gemv_dot_kernel<1, 1, 4, 8, true, true>", 20_000, 3),
                         ("gemv_mfma_kernel<1, 1, 2, 8, true, true, true>", 21_000, 2),   # M = 2
                         ("gemv_dot_kernel<2, 1, 2, 16, true, false>", 5_000, 1),          # M = 2, only M = 2 uses it
                         ("gemv_mfma_kernel<1, 2, 2, 16, false, true, false>", 7_000, 1),  # M = 4, only M = 4
                         ("gemv_mfma_kernel<1, 1, 2, 8, true, true, true>", 23_000, 2)):  # M = 4
        for _ in range(n):
            g, wg = (229376, 1024) if "<2, 1, 2, 16" in name else (36864, 256) if "<1, 2, 2" in name else (grid, 256)
            trace.append({"Kernel_Name": f"void tf::(anonymous namespace)::{name}(tf::LinearArgs, int)",
                          "Start_Timestamp": t, "End_Timestamp": t + dur, "Grid_Size_X": g,
                          "Workgroup_Size_X": wg})
            t += dur + 1000
    with open(d / "1_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(trace[0]))
        w.writeheader()
        w.writerows(trace)
    o2 = {"kernel": "gemv_dot", "block_m": 2, "block_n": 16, "block_k": 128, "split_k": 1, "num_warps": 16,
          "num_stages": 2}
    line = {"metric": "m", "per_shape": [{"layer": "gate_up_proj", "m": 1, "us": 20.5, "config": dot}],
            "gemv_m2_m4": [{"layer": "gate_up_proj", "m": 2, "us": 21.2, "config": mfma},
                           {"layer": "o_proj", "m": 2, "us": 5.1, "config": o2},
                           {"layer": "qkv_proj", "m": 4, "us": 7.2,
                            "config": dict(mfma, block_n=32, block_k=64, num_warps=4)},
                           {"layer": "gate_up_proj", "m": 4, "us": 22.9, "config": mfma}],
            "gemm_m256": []}
    log = tmp_path / "bench.log"
    log.write_text("noise\n" + json.dumps(line) + "\n")
    assert bench.stats_summary(str(tmp_path / "prof"), str(log)) == 0
    text = (tmp_path / "stats.md").read_text()
    assert "| gate_up_proj M=1 | `gemv_dot_kernel<1, 1, 4, …, true, true>` | 151552 | 3 | 20.00 | 20.50 |" in text
    assert "| gate_up_proj M=2 | `gemv_mfma_kernel<1, 1, 2, …, true, true, true>` | 151552 | 2 | 21.00 | 21.20 |" in text
    assert "| gate_up_proj M=4 | `gemv_mfma_kernel<1, 1, 2, …, true, true, true>` | 151552 | 2 | 23.00 | 22.90 |" in text
