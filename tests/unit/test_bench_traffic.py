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
        rows.append({"Dispatch_Id": did, "Kernel_Name": "void tf::gemv_kernel<1, 1, 2, 16, true, false, 1>(...)",
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
    assert "| gemv_dot bm1 bn16 bk128 sk1 w4 st2 |" in text
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
                     "GRBM_GUI_ACTIVE": cycles * bench.NUM_XCDS, "SQ_INSTS_LDS": 1000.0,
                     "SQ_LDS_BANK_CONFLICT": 500.0}.get(c, 1.0)
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
    assert ("| gate_up_proj | W4A16 fp16 | gemm_mfma bm256 bn192 bk64 sk1 w8 st3 | 30.0% | 100.00 | 700.0 | "
            "28.0% of 2.5 PF | 0.50 |") in text
    assert "| down_proj | W4A16 fp16 | gemm_mfma bm256 bn192 bk64 sk1 w8 st3 | 20.0% |" in text


def _marked_trace(groups: list, t0: int = 0) -> list:  # type: ignore[type-arg]
    """A kernel trace: setup kernels, then each group's dispatches after a marker kernel, then
    the calibration kernel (file order reversed: the summary orders by dispatch id)."""
    trace, did, t = [], 1, t0
    names = [("fill_kernel", 1000)]
    for g in groups:
        names += [("bitwise_not_kernel", 500)] + g
    names += [("bitwise_not_kernel", 500), ("neg_kernel", 9000)]
    for name, dur in names:
        trace.append({"Dispatch_Id": did, "Kernel_Name": f"void tf::(anonymous namespace)::{name}(tf::LinearArgs, int)",
                      "Start_Timestamp": t, "End_Timestamp": t + dur})
        did, t = did + 1, t + dur + 1000
    trace.reverse()
    return trace


def test_stats_summary_sums_each_ops_kernels_between_markers(tmp_path: Path,
                                                            monkeypatch: pytest.MonkeyPatch) -> None:
    """--stats-summary: the kernel table comes from the bench trace; the entry probe's dispatches
    between marker kernels are one op's launches, and an op's time per launch is the sum over
    its kernels (a split-K GEMM and its reduce), set beside the bench's event-timed average."""
    out = tmp_path / "stats.md"
    monkeypatch.setattr(bench, "STATS_SUMMARY", out)
    d = tmp_path / "prof" / "vm"
    d.mkdir(parents=True)
    with open(d / "1_kernel_stats.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Name", "Calls", "AverageNs", "MinNs", "MaxNs", "Percentage"])
        w.writeheader()
        w.writerow({"Name": "void tf::(anonymous namespace)::gemv_kernel<1, 1, 2, 16, true, false, 1>(tf::LinearArgs, int)",
                    "Calls": 3, "AverageNs": 20000, "MinNs": 19000, "MaxNs": 21000, "Percentage": 50.0})
    gemm = {"kernel": "gemm_mfma", "block_m": 128, "block_n": 256, "block_k": 64, "split_k": 8, "num_warps": 8,
            "num_stages": 3}
    entries = [{"entry": "gate_up_proj M=1", "config": CFGS[0], "bytes": 1},
               {"entry": "down_proj M=256", "config": gemm, "bytes": 1}]
    launches = 2
    trace = _marked_trace([[("gemv_kernel<1, 1, 2, 16, true, false, 1>", 20_000),
                            ("gemv_kernel<1, 1, 2, 16, true, false, 1>", 22_000)],
                           [("gemm2_kernel<128, 256, 4, 2, 3>", 60_000), ("splitk_reduce_kernel", 8_000),
                            ("gemm2_kernel<128, 256, 4, 2, 3>", 64_000), ("splitk_reduce_kernel", 8_000)]])
    k = tmp_path / "kprof" / "vm"
    k.mkdir(parents=True)
    with open(k / "2_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(trace[0]))
        w.writeheader()
        w.writerows(trace)
    line = {"metric": "m", "per_shape": [{"layer": "gate_up_proj", "m": 1, "us": 20.5, "config": CFGS[0]}],
            "gemv_m2_m4": [], "gemm_m256": [{"layer": "down_proj", "m": 256, "us": 70.0, "config": gemm}],
            "gemm_m1024_m4096": []}
    log = tmp_path / "bench.log"
    log.write_text("noise\n" + json.dumps(line) + "\n")
    kp = tmp_path / "entries.log"
    kp.write_text(json.dumps({"entry_probe": {"launches": launches, "entries": entries}}) + "\n")
    args = [str(tmp_path / "prof"), str(log), str(log), str(tmp_path / "kprof"), str(kp)]
    assert bench.stats_summary(*args) == 0
    text = out.read_text()
    assert ("| gate_up_proj M=1 | gemv_dot bm1 bn16 bk128 sk1 w4 st2 | `tf::gemv_kernel<1, 1, 2, 16, true, false, 1>` "
            "| 21.00 | 20.50 | 1.02 |") in text
    assert ("| down_proj M=256 | gemm_mfma bm128 bn256 bk64 sk8 w8 st3 | `tf::gemm2_kernel<128, 256, 4, 2, 3>`, "
            "`tf::splitk_reduce_kernel` | 70.00 | 70.00 | 1.00 |") in text
    # A probe run on another config is refused.
    kp.write_text(json.dumps({"entry_probe": {"launches": launches, "entries": [dict(entries[0], config=CFGS[1]),
                                                                                entries[1]]}}) + "\n")
    out.unlink()
    assert bench.stats_summary(*args) == 1
    assert not out.exists()


def test_counter_summary_sums_each_ops_kernels(tmp_path: Path, monkeypatch: pytest.MonkeyPatch) -> None:
    """--counter-summary: FETCH/WRITE KiB of every dispatch between two markers, summed per launch
    and scaled by the calibration kernel's known / counted bytes."""
    out = tmp_path / "traffic.md"
    monkeypatch.setattr(bench, "ENTRY_TRAFFIC_SUMMARY", out)
    entries = [{"entry": "down_proj M=256", "config": CFGS[0], "bytes": 4096},
               {"entry": "rmsnorm_fp8 T=4096", "bytes": 2048}]
    for counter, sub in (("FETCH_SIZE", "f"), ("WRITE_SIZE", "w")):
        d = tmp_path / sub
        d.mkdir()
        trace = _marked_trace([[("gemm2_kernel", 1), ("splitk_reduce_kernel", 1)] * 2, [("rmsnorm_kernel", 1)] * 2])
        rows = [{"Dispatch_Id": r["Dispatch_Id"], "Kernel_Name": r["Kernel_Name"], "Counter_Name": counter,
                 "Counter_Value": 2.0 if "gemm2" in r["Kernel_Name"] else 1.0 if "reduce" in r["Kernel_Name"] else
                 (131072.0 if "neg" in r["Kernel_Name"] else 1.0)} for r in trace]
        with open(d / "pmc_counter_collection.csv", "w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=list(rows[0]))
            w.writeheader()
            w.writerows(rows)
    log = tmp_path / "probe.log"
    log.write_text(json.dumps({"entry_probe": {"launches": 2, "entries": entries,
                                                "calibration_bytes_in": 256 << 20}}) + "\n")
    assert bench.counter_summary(str(tmp_path / "f"), str(tmp_path / "w"), str(log)) == 0
    text = out.read_text()
    # 256 MiB known / 128 MiB counted = scale 2; the GEMM launch is 3 KiB counted -> 6144 bytes.
    assert "| down_proj M=256 | gemv_dot bm1 bn16 bk128 sk1 w4 st2 | 6144 | 6144 | 12288 | 4096 | 3.000 |" in text
    assert "| rmsnorm_fp8 T=4096 | - | 2048 | 2048 | 4096 | 2048 | 2.000 |" in text


def _bench_log(path: Path, cfg: dict) -> str:  # type: ignore[type-arg]
    line = {"metric": "m", "per_shape": [{"layer": "gate_up_proj", "m": 1, "us": 18.0, "config": cfg}],
            "gemm_m256": [], "gemm_m1024_m4096": []}
    path.write_text("setup\n" + json.dumps(line) + "\n")
    return str(path)


def test_stats_summary_refuses_runs_on_different_configs(tmp_path: Path, monkeypatch: pytest.MonkeyPatch) -> None:
    out = tmp_path / "stats.md"
    monkeypatch.setattr(bench, "STATS_SUMMARY", out)
    a = _bench_log(tmp_path / "a.log", CFGS[0])
    b = _bench_log(tmp_path / "b.log", CFGS[1])
    assert bench.stats_summary(str(tmp_path / "prof"), a, b, str(tmp_path / "kprof"), a) == 1
    assert not out.exists()


def test_probe_summary_table(tmp_path: Path, monkeypatch: pytest.MonkeyPatch) -> None:
    out = tmp_path / "floors.md"
    monkeypatch.setattr(bench, "PROBE_SUMMARY", out)
    rows = [{"probe": "empty", "grid": 256, "us": 1.6}]
    for name, n, k in bench.SHAPES:
        rows += [{"probe": "gemv", "layer": name, "config": CFGS[0], "us": 20.0, "gbps": 4000.0, "tuned": True},
                 {"probe": "gemv", "layer": name, "config": CFGS[1], "us": 19.0, "gbps": 4200.0, "tuned": False}]
        for pat, us in (("tile", 14.0), ("tile+meta", 15.0), ("rows", 17.0), ("stream", 13.0)):
            rows += [{"probe": pat, "layer": name, "waves": 4, "depth": 4, "us": us, "gbps": 5000.0},
                     {"probe": pat, "layer": name, "waves": 8, "depth": 2, "us": us + 1, "gbps": 4000.0}]
        for pat, us in (("wave", 16.0), ("group", 12.5), ("grid", 12.0)):
            rows += [{"probe": pat, "layer": name, "grid": 512, "waves": 8, "depth": 2, "us": us, "gbps": 5600.0},
                     {"probe": pat, "layer": name, "grid": 256, "waves": 16, "depth": 4, "us": us + 2, "gbps": 4800.0}]
    log = tmp_path / "probe.log"
    log.write_text(json.dumps({"read_probe": rows}) + "\n")
    assert bench.probe_summary(str(log)) == 0
    text = out.read_text()
    # in use, best candidate, best K-split candidate (CFGS[1] has block_k 128), then the floors
    assert ("| gate_up_proj 37888x3584 | 20.00 (4000 GB/s) | 19.00 (4200 GB/s) | 19.00 (4200 GB/s) | "
            "14.00 (5000 GB/s) |") in text
    assert "| 1.60 |" in text  # in use / group: 20 / 12.5
    assert "group grid 512 w8 d2" in text
