"""Benchmark of the MI355X quantized-linear hot path (one JSON result line on stdout).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--tune] [--no-cpu] [--detail PATH] [--full]
                    [--no-stack] [--check] [--update-baseline [PATH] --reason TEXT]
    python bench.py --fingerprint        (the environment fingerprint of this checkout)
    python bench.py --traffic-probe      (eager launches for rocprofv3 --pmc, see below)
    python bench.py --mfma-probe         (the M=256 GEMMs, for rocprofv3 --pmc)
    python bench.py --entry-probe        (eager launches of every timed op, for rocprofv3)
    python bench.py --probe              (memory floors of the GEMV's access patterns)
    python bench.py --traffic-summary FETCH_DIR WRITE_DIR PROBE_LOG   (write the profiles/ summaries
    python bench.py --mfma-summary PMC_DIR PROBE_LOG TIMING_LOG        from the profiler's output)
    python bench.py --stats-summary PROF_DIR BENCH_LOG PROF_LOG KPROF_DIR KPROBE_LOG
    python bench.py --counter-summary FETCH_DIR WRITE_DIR PROBE_LOG
    python bench.py --instr-summary PMC_DIR PROBE_LOG
    python bench.py --probe-summary PROBE_LOG

Configs: every timed launch uses the config ``autotune.lookup`` returns, i.e. the autotune
cache, else the table shipped for this GPU in ``tokenforge/kernels/tuned/``, else the heuristic
default; each JSON entry carries its ``config`` and ``config_source``. ``--tune`` first retunes
every timed shape and bucket into the cache (as process_weights_after_loading would); that is
how the shipped table is made. The committed profiles are made with the same configs as the
bench line, and the summary steps refuse to write when the runs they combine used different
ones.

Workload (BASELINE.json metric "W4A16 GEMV HBM GB/s at M=1 + GEMM TFLOP/s at M=256"):
one step is one decode pass at M=1 through the four Qwen2.5-7B decoder linears (qkv
4608x3584, o_proj 3584x3584, gate_up 37888x3584, down 3584x18944; configs[2] at M=1) with
AWQ int4 group-128 weights: nibbles and zero-points uniform in [0, 15], fp16 scales uniform
in [1e-3, 1e-2], x ~ N(0, 1) fp16. Ten layer copies (1.21 GB) rotate so every step reads its
weights from HBM, not from the 256 MB Infinity Cache. Weights are built in AWQ format and
converted with the GPU repack (AWQ -> TokenForge layout -> gfx950 tile layout) before anything
is timed.

``value`` = algorithmic bytes of the K timed steps (micro.py:82-86 formula, summed over the
four linears) / wall time of the K steps, in GB/s. The steps are replayed from a HIP graph
so host launch overhead is not measured; inputs are resident in HBM. Per-kernel figures
(``per_shape``, ``gemm_m256``, ``rmsnorm_fp8``, ``gemm_sweep``) are the median over 5 replays
of a graph of launches rotating over the cold copies.

Extra objects on the same JSON line:
* ``roofline``: the dominant kernel (gate_up GEMV, M=1): algorithmic bytes per launch / its
  average launch duration, timed with HIP events on the stream it is launched on, against the
  8 TB/s HBM peak. ``traffic`` is the HBM bytes per launch that rocprofv3 counted
  (FETCH_SIZE + WRITE_SIZE, each scaled by the ratio of known bytes to counted bytes of a
  plain elementwise kernel in the same run), read from the committed summary
  ``profiles/gemv_gate_up_m1_traffic.md``, which holds one row per autotune candidate of the
  gate_up M=1 bucket (null if the config in use has no row). ``--traffic-probe`` runs exactly
  what those counter passes measure: every candidate in turn on the rotating cold copies, then
  the calibration kernel (torch.neg, 256 MiB in and out); ``--traffic-summary FETCH_DIR
  WRITE_DIR PROBE_LOG`` turns the two counter runs into that summary.
* ``gemm_small_m``, ``gemm_m256`` and ``gemm_m1024_m4096``: the GEMM at M = 16,
  32, 64, 128, 256, 1024 and 4096 on gate_up and down (x ~ N(0, 1) fp16 with 1% of the rows
  scaled by 10), TFLOP/s and fraction of the 2.5 PFLOP/s fp16 dense MFMA peak; each entry is
  the whole op (a split-K launch and its reduce kernel are both in the graph).
* ``gemm_w4a8_fp8``: the W4A8 linear at the same M and shapes on e4m3 activations with per-row
  scales, run by the fp8-MFMA GEMM the op picks there (``fp8_gemm_config``), TFLOP/s against
  the 2.5 PF fp16 and 5 PF fp8 dense peaks.
* ``repack_gate_up``: the load-time AWQ -> TokenForge repack (pack.py:141-143) of gate_up's
  qweight, int4 values per second (and the bytes read + written per second).
* ``device_copy_gbps``: the box's achievable bandwidth of a plain device copy (torch, 1 GiB
  read and written), read + write bytes per second, next to the 8 TB/s peak.
* ``per_shape`` and ``gemv_m2_m4``: the GEMV on each of the four shapes at
  M = 1, and at M = 2 and 4 (buckets 2 and 4 autotuned), average launch duration and GB/s;
  ``gemv_m8_m32``: the same four shapes at M = 8 and 32, the rest of the reference's l4 suite
  (micro.py:58, M in {1, 8, 32}).
* ``vendor_fp16``: the vendor's dense fp16 linear beside them, as micro.py:110-114 runs
  ``cublas-fp16`` beside every case: ``torch.nn.functional.linear`` with fp16 weights
  (hipBLASLt) on the four shapes at M in {1, 8, 32} and on gate_up and down at M = 256, 1024
  and 4096, weights rotating over >= 1.1 GB of copies; GB/s with the dense byte count.
* ``eager_op``: the M=1 op called eagerly, back to back, without a graph (micro.py:67-79's
  method): per call, the stream's time (HIP events) and the host's time to issue it, for the
  custom op and for the launcher under it.
* ``rmsnorm_fp8``: the fused RMSNorm + e4m3fn quant (configs[1]: H=3584, eight outlier
  channels x20, gamma = 1 + 0.1 N(0,1), eps 1e-6, dynamic per-token scale) at T in
  {1, 16, 512, 4096}; algorithmic bytes T*H*2 + H*2 + T*H + 4*T over rotating cold inputs;
  ``us`` is the form the hot path picks, ``us_by_form`` each kernel form (row per workgroup,
  row per wave).
* with ``--full`` only (written to ``--detail``): ``gemm_sweep``, configs[3]: M in
  {16, 32, 64, 128, 256, 1024, 4096} on gate_up and down (configs as above); and
  ``vendor_fp16_gemm``, the vendor's dense fp16 GEMM (torch.matmul, hipBLASLt) on the same
  shapes at M in {256, 1024, 4096} with fp16 weights, as a reference point for the MFMA
  fraction this box reaches on these shapes.
* ``stack``: 28 Qwen2.5-7B decoder layers of distinct synthetic weights (3.39 GB
  int4 + scales + zeros; qkv with an fp16 bias), one pass per step: RMSNorm + FP8 -> fp16(q *
  scale) -> qkv -> attention as identity on the value slice (query head h takes KV group
  h // 7) -> o_proj -> residual add -> RMSNorm + FP8 -> fp16(q * scale) -> gate_up -> SiLU(gate)
  * up -> down -> residual add. The linears and the norms are this library's kernels, the
  rest is torch glue ("unfused"), or the residual adds and SiLU*mul run as the linears'
  fused epilogues and each norm with fp16(q * scale) runs inside the linear that reads it
  (rmsnorm_fp8_w4a16_linear: the decode GEMV's prologue at M <= 4, the norm kernel writing
  fp16(q * scale) itself above) ("fused", same bits; ``tokens_per_s`` is this one), or in
  addition qkv and
  gate_up take the FP8 codes and scales directly as W4A8 linears ("w4a8", no fp16(q * scale)
  glue; not bit-equal: the scale multiplies each row's sum instead of each element; from M = 128
  these run on the fp8-MFMA GEMM, which also applies the group scale exactly). A pass
  is one HIP graph, tokens/s = M / time per pass, at M in {1, 8, 32} (decode) and 2048
  (prefill).
* ``cpu_baseline``: reference.py's CPU path (dequantize per call + fp32 matmul), restated in
  torch on the host cores (``oracle/cpu_path.py``), on a bounded sample of the same step, with
  the host CPU's model name and the threads used. The same restatements are timed beside the
  M=16 and M=256 GEMMs (``gemm_small_m[i].cpu``, ``gemm_m256[i].cpu``), the M=8 decode step
  (``cpu_decode_m8``), the RMSNorm + FP8 at T=4096 (``rmsnorm_fp8[..].cpu``) and the repack
  (``repack_gate_up.cpu``). The stack has none: one CPU pass of 28 layers takes ~12 s per token.
* ``env``: the environment fingerprint (env.py:51-85): git commit and dirty flag (null in a
  copy without ``.git``, such as the GPU box's), the sha256 code-tree hash of the sources under
  ``CODE_PATHS`` (``--fingerprint`` prints it for a checkout), torch, HIP, the library's ABI,
  the GPU.
* ``regression``: every timed entry against the committed baseline for this GPU
  (``bench_baseline.json``, written by ``--update-baseline --reason``; micro.py:140-181): the
  entries more than 5% slower and the headline's ratio to the baseline's. ``--check`` exits 1
  on a regression. The top-level ``vs_baseline`` stays null: it is reserved for a published
  number for this metric, and the reference publishes none.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

HBM_PEAK_GBPS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0
FP8_MFMA_PEAK_TFLOPS = 5000.0
GROUP = 128
SHAPES = [  # (layer, N, K)
    ("qkv_proj", 4608, 3584),
    ("o_proj", 3584, 3584),
    ("gate_up_proj", 37888, 3584),
    ("down_proj", 3584, 18944),
]
COLD_BYTES = 1.1e9
TRAFFIC_SUMMARY = ROOT / "profiles" / "gemv_gate_up_m1_traffic.md"
MFMA_SUMMARY = ROOT / "profiles" / "gemm_m256_mfma_busy.md"
STATS_SUMMARY = ROOT / "profiles" / "bench_decode_m1_kernel_stats.md"
MFMA_COUNTERS = ("SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE", "SQ_BUSY_CYCLES", "SQ_WAVES", "SQ_INSTS_LDS",
                 "SQ_ACTIVE_INST_LDS", "SQ_LDS_BANK_CONFLICT")
NUM_SIMDS = 256 * 4
NUM_XCDS = 8
CALIB_BYTES = 256 << 20
COPY_BYTES = 1 << 30
MFMA_LAUNCHES = 8
PREFILL_M = (256, 1024, 4096)
SMALL_M = (16, 32, 64, 128)  # configs[3] below the prefill M
DECODE_EXTRA_M = (8, 32)  # the reference's l4 suite (micro.py:58): M in {1, 8, 32}
SWEEP_M = (16, 32, 64, 128, 256, 1024, 4096)
STACK_M = (1, 8, 32, 2048)
BASELINE_FILE = ROOT / "bench_baseline.json"
REGRESSION = 0.05  # micro.py:30: an entry more than 5% slower than the committed baseline
# Files whose content a bench line vouches for (the code-tree hash of the fingerprint).
CODE_PATHS = ("bench.py", "__graft_entry__.py", "tokenforge", "tokenforge_amd", "include", "bench_probes")
CODE_SUFFIXES = (".py", ".hip", ".h", ".json")
NORM_H = 3584
NORM_T = (1, 16, 512, 4096)
TIMED_SECTIONS = ("per_shape", "gemv_m2_m4", "gemv_m8_m32", "gemm_small_m", "gemm_m256", "gemm_m1024_m4096")


def committed_traffic(cfg_dict: dict) -> float | None:  # type: ignore[type-arg]
    """HBM bytes per launch of the dominant kernel with config ``cfg_dict`` from the committed
    counter summary; its lines ``traffic: <bytes per launch> <config json>`` carry one config
    each."""
    if not TRAFFIC_SUMMARY.is_file():
        return None
    for line in TRAFFIC_SUMMARY.read_text().splitlines():
        if not line.startswith("traffic: "):
            continue
        try:
            value, cfg = line[len("traffic: "):].split(" ", 1)
            if json.loads(cfg) == cfg_dict:
                return float(value)
        except ValueError:
            return None
    return None


def traffic_summary(fetch_dir: str, write_dir: str, probe_log: str) -> int:
    """Write ``TRAFFIC_SUMMARY`` from two ``rocprofv3 --pmc`` runs of ``--traffic-probe`` (one
    with FETCH_SIZE, one with WRITE_SIZE) and the probe's own output line. The GEMV dispatches
    of each run are grouped in launch order, ``launches`` per candidate; each counter is scaled
    by known bytes / counted bytes of the calibration kernel in the same run."""
    import csv
    import glob

    probe = None
    for line in Path(probe_log).read_text().splitlines():
        if line.startswith('{"traffic_probe"'):
            probe = json.loads(line)["traffic_probe"]
    if probe is None:
        print(f"no traffic_probe line in {probe_log}", file=sys.stderr)
        return 1

    def counter(d: str, name: str) -> tuple[list, float]:  # type: ignore[type-arg]
        rows = []
        for f in glob.glob(f"{d}/**/*counter_collection.csv", recursive=True):
            rows += [r for r in csv.DictReader(open(f)) if r["Counter_Name"] == name]
        rows.sort(key=lambda r: int(r["Dispatch_Id"]))
        gemv = [float(r["Counter_Value"]) * 1024 for r in rows if "gemv_" in r["Kernel_Name"]]
        calib = [float(r["Counter_Value"]) * 1024 for r in rows if "neg_kernel" in r["Kernel_Name"]]
        if not calib or len(gemv) != probe["launches"] * len(probe["configs"]):
            raise ValueError(f"{d}: {len(gemv)} GEMV dispatches, {len(calib)} calibration dispatches")
        return gemv, probe["calibration_bytes_in"] / statistics.mean(calib)

    fetch, f_scale = counter(fetch_dir, "FETCH_SIZE")
    write, w_scale = counter(write_dir, "WRITE_SIZE")
    n_launch = probe["launches"]
    alg = probe["algorithmic_bytes"]
    lines = [
        "# HBM traffic of the dominant kernel: gate_up GEMV at M=1 (37888 x 3584, g128)",
        "",
        "Commands (on the MI355X box; one counter per run, each run a separate process):",
        "",
        "```",
        "cd /tmp && export TMPDIR=/tmp && R=<repo root>",
        "timeout -s KILL 150 rocprofv3 --pmc FETCH_SIZE --output-format csv -d $R/gpurun_out/pmc_fetch -- \\",
        "    python $R/bench.py --traffic-probe > $R/gpurun_out/pmc_fetch.log",
        "timeout -s KILL 150 rocprofv3 --pmc WRITE_SIZE --output-format csv -d $R/gpurun_out/pmc_write -- \\",
        "    python $R/bench.py --traffic-probe > $R/gpurun_out/pmc_write.log",
        "python $R/bench.py --traffic-summary $R/gpurun_out/pmc_fetch $R/gpurun_out/pmc_write \\",
        "    $R/gpurun_out/pmc_fetch.log",
        "```",
        "",
        f"`--traffic-probe` launches every autotune candidate of the gate_up M=1 bucket {n_launch} times",
        "over the rotating cold layer copies, then the calibration kernel `torch.neg` on a 256 MiB",
        "fp32 tensor (256 MiB read, 256 MiB written) 4 times. Counters are KiB per dispatch;",
        f"scale = known / counted bytes of the calibration kernel: FETCH_SIZE x {f_scale:.4f},",
        f"WRITE_SIZE x {w_scale:.4f}. Algorithmic bytes per launch (weights N*K/2 + scales + zero",
        f"points + x + y): {alg}. Rows: mean over the launches of each candidate.",
        "",
        "| config | FETCH bytes | WRITE bytes | traffic / launch | x algorithmic |",
        "|---|---:|---:|---:|---:|",
    ]
    machine = []
    for i, cfg in enumerate(probe["configs"]):
        fb = statistics.mean(fetch[i * n_launch:(i + 1) * n_launch]) * f_scale
        wb = statistics.mean(write[i * n_launch:(i + 1) * n_launch]) * w_scale
        t = fb + wb
        name = (f"{cfg['kernel']} bm{cfg['block_m']} bn{cfg['block_n']} bk{cfg['block_k']} "
                f"sk{cfg['split_k']} w{cfg['num_warps']} st{cfg['num_stages']}")
        lines.append(f"| {name} | {fb:.0f} | {wb:.0f} | {t:.0f} | {t / alg:.3f} |")
        machine.append(f"traffic: {t:.0f} {json.dumps(cfg)}")
    lines += ["", "Machine-readable (bench.py reads the row of the config in use):", "", "```", *machine, "```", ""]
    TRAFFIC_SUMMARY.write_text("\n".join(lines))
    print(f"wrote {TRAFFIC_SUMMARY} ({len(probe['configs'])} configs)")
    return 0


def _bench_line(log_path: str) -> dict | None:  # type: ignore[type-arg]
    bench = None
    for line in Path(log_path).read_text().splitlines():
        if line.startswith("{") and '"metric"' in line:
            bench = json.loads(line)
    return bench


def _configs_of(bench: dict) -> dict:  # type: ignore[type-arg]
    """(section, layer, M) -> config of every timed kernel entry of a bench JSON line."""
    out = {}
    for sec in TIMED_SECTIONS:
        for e in bench.get(sec) or []:
            out[(sec, e["layer"], e["m"])] = e["config"]
    return out


MARKER_KERNEL = "bitwise_not"  # the entry probe's separator kernel (torch.bitwise_not on one int)
CALIB_KERNEL = "neg_kernel"  # the entry probe's calibration kernel (torch.neg, known bytes)
ENTRY_TRAFFIC_SUMMARY = ROOT / "profiles" / "hbm_traffic_per_entry.md"
INSTR_SUMMARY = ROOT / "profiles" / "instruction_mix_per_entry.md"
INSTR_COUNTERS = ("SQ_WAVES", "SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_LDS", "SQ_INSTS_VMEM_RD", "SQ_INSTS_SALU",
                  "SQ_BUSY_CYCLES", "GRBM_GUI_ACTIVE")
def marker_groups(rows: list, entries: int) -> list[list]:  # type: ignore[type-arg]
    """Split an entry probe's dispatches (dicts with ``Dispatch_Id`` and ``Kernel_Name``) into
    one list per entry: the dispatches between consecutive marker kernels, in dispatch order
    (what follows the last marker is the calibration's setup and the calibration kernel). Rows
    that share a dispatch (one per counter) stay together."""
    order = sorted({int(r["Dispatch_Id"]) for r in rows})
    by_id: dict = {}  # type: ignore[type-arg]
    for r in rows:
        by_id.setdefault(int(r["Dispatch_Id"]), []).append(r)
    groups: list[list] = []  # type: ignore[type-arg]
    current = None
    for did in order:
        name = by_id[did][0]["Kernel_Name"]
        if MARKER_KERNEL in name:
            if current is not None:
                groups.append(current)
            current = []
        elif CALIB_KERNEL in name:
            break
        elif current is not None:
            current.extend(by_id[did])
    if len(groups) != entries:
        raise ValueError(f"{len(groups)} marked groups of dispatches, expected {entries}")
    return groups


def _event_times(bench: dict) -> dict:  # type: ignore[type-arg]
    """Entry name -> (event-timed us, config) of a bench JSON line's timed entries."""
    out = {}
    for sec in TIMED_SECTIONS:
        for e in bench.get(sec) or []:
            out[f"{e['layer']} M={e['m']}"] = (e["us"], e.get("config"))
    for e in bench.get("gemm_w4a8_fp8") or []:
        out[f"{e['layer']} M={e['m']} W4A8"] = (e["us"], e.get("config"))
    for e in bench.get("rmsnorm_fp8") or []:
        out[f"rmsnorm_fp8 T={e['t']}"] = (e["us"], None)
    if bench.get("repack_gate_up"):
        out["repack gate_up_proj"] = (bench["repack_gate_up"]["us"], None)
    return out


def _short(name: str) -> str:
    name = name.replace("(anonymous namespace)::", "").replace("void ", "")
    return name.split("(tf::")[0].split("(unsigned")[0].split("(int")[0].split("(float")[0].split("(long")[0]


def _cfg_name(c: dict | None) -> str:  # type: ignore[type-arg]
    if not c:
        return "-"
    return (f"{c['kernel']} bm{c['block_m']} bn{c['block_n']} bk{c['block_k']} sk{c['split_k']} "
            f"w{c['num_warps']} st{c['num_stages']}")


def stats_summary(prof_dir: str, bench_log: str, prof_log: str, kprof_dir: str, kprobe_log: str) -> int:
    """Write ``STATS_SUMMARY`` from two ``rocprofv3 --kernel-trace --stats`` runs: one of the
    bench itself (``prof_dir``, its stdout in ``prof_log``: the kernel table) and one of
    ``--entry-probe`` (``kprof_dir``, stdout in ``kprobe_log``: each timed op's launches between
    marker kernels), next to the event-timed averages of the plain bench run before them
    (``bench_log``). An op's time is the sum of all its kernels per launch (a split-K GEMM and
    its reduce). Refuses to write when the runs used different configs for any timed shape."""
    import csv
    import glob

    bench, prof = _bench_line(bench_log), _bench_line(prof_log)
    probe = _probe_line(kprobe_log, "entry_probe")
    if bench is None or prof is None or probe is None:
        print(f"no bench JSON line in {bench_log} or {prof_log}, or no entry_probe line in {kprobe_log}",
              file=sys.stderr)
        return 1
    cb, cp = _configs_of(bench), _configs_of(prof)
    ev = _event_times(bench)
    ck = {e["entry"]: e.get("config") for e in probe["entries"]}
    differ = sorted(str(key) for key in set(cb) & set(cp) if cb[key] != cp[key])
    differ += sorted(name for name, c in ck.items() if c is not None and name in ev and ev[name][1] is not None
                     and ev[name][1] != c)
    if differ or not set(cb) & set(cp):
        print(f"the bench, profiled and probe runs used different configs: {differ}", file=sys.stderr)
        return 1
    PRE = "cd /tmp && export TMPDIR=/tmp && R=<repo root>"
    # ---------------------------------------------------------------- kernel stats
    f = glob.glob(f"{prof_dir}/**/*_kernel_stats.csv", recursive=True)[0]
    rows = list(csv.DictReader(open(f)))
    lines = [
        "# Kernel statistics of the bench, and each timed op's rocprofv3 time beside its event timing",
        "",
        "Commands (on the MI355X box, fresh autotune cache, so every run takes its configs from",
        "the table shipped in tokenforge/kernels/tuned/; the summary step checks that they agree):",
        "",
        "```",
        PRE,
        "python $R/bench.py --no-cpu > $R/gpurun_out/bench.log",
        "rocprofv3 --kernel-trace --stats --output-format csv -d $R/gpurun_out/prof_bench -- \\",
        "    python $R/bench.py --steps 20 --warmup 5 --no-cpu --no-stack > $R/gpurun_out/prof_bench.log",
        "rocprofv3 --kernel-trace --stats --output-format csv -d $R/gpurun_out/prof_entries -- \\",
        "    python $R/bench.py --entry-probe > $R/gpurun_out/entries.log",
        "python $R/bench.py --stats-summary $R/gpurun_out/prof_bench $R/gpurun_out/bench.log \\",
        "    $R/gpurun_out/prof_bench.log $R/gpurun_out/prof_entries $R/gpurun_out/entries.log",
        "```",
        "",
        "Kernel table: `*_kernel_stats.csv` of the profiled bench run (graph replays of every timed",
        "entry, the warmups and the setup kernels), the 24 kernels with the most time.",
        "",
        "| kernel | calls | avg us | min us | max us | % time |",
        "|---|---:|---:|---:|---:|---:|",
    ]
    for r in rows[:24]:
        name = _short(r["Name"])
        if len(name) > 90:
            name = name[:90] + "..."
        lines.append(f"| `{name}` | {r['Calls']} | {float(r['AverageNs'])/1e3:.2f} | {float(r['MinNs'])/1e3:.2f} | "
                     f"{float(r['MaxNs'])/1e3:.2f} | {float(r['Percentage']):.1f} |")
    # ---------------------------------------------------------------- per entry
    tr = glob.glob(f"{kprof_dir}/**/*_kernel_trace.csv", recursive=True)[0]
    groups = marker_groups(list(csv.DictReader(open(tr))), len(probe["entries"]))
    n_launch = probe["launches"]
    lines += [
        "",
        f"Per op: the `--entry-probe` trace, each op launched {n_launch} times eagerly on the rotating",
        "cold copies between two marker kernels; rocprofv3 time per launch summed over all the op's",
        "kernels (a split-K GEMM and its reduce both count), next to the event-timed average of the",
        "plain bench run (HIP events around graph replays on the launch stream).",
        "",
        "| op | config | kernels per launch | rocprofv3 us / launch | event-timed us | ratio |",
        "|---|---|---|---:|---:|---:|",
    ]
    for e, ds in zip(probe["entries"], groups):
        if len(ds) % n_launch:
            raise ValueError(f"{e['entry']}: {len(ds)} dispatches for {n_launch} launches")
        per = statistics.mean((int(d["End_Timestamp"]) - int(d["Start_Timestamp"])) / 1e3 for d in ds) * len(ds) / n_launch
        kinds: dict = {}  # type: ignore[type-arg]
        for d in ds:
            kinds[_short(d["Kernel_Name"])] = kinds.get(_short(d["Kernel_Name"]), 0) + 1
        kern = ", ".join(f"`{k}`" + (f" x{v // n_launch}" if v // n_launch > 1 else "") for k, v in kinds.items())
        t = ev.get(e["entry"])
        ev_us = f"{t[0]:.2f}" if t else "-"
        ratio = f"{per / t[0]:.2f}" if t else "-"
        lines.append(f"| {e['entry']} | {_cfg_name(e.get('config'))} | {kern} | {per:.2f} | {ev_us} | {ratio} |")
    STATS_SUMMARY.write_text("\n".join(lines) + "\n")
    print(f"wrote {STATS_SUMMARY}")
    return 0


def counter_summary(fetch_dir: str, write_dir: str, probe_log: str) -> int:
    """Write ``ENTRY_TRAFFIC_SUMMARY`` from two ``rocprofv3 --pmc`` runs of ``--entry-probe``
    (FETCH_SIZE, then WRITE_SIZE): each op's HBM bytes per launch (all its kernels), each
    counter scaled by known bytes / counted bytes of the calibration kernel in the same run,
    next to the op's algorithmic bytes."""
    import csv
    import glob

    probe = _probe_line(probe_log, "entry_probe")
    if probe is None:
        print(f"no entry_probe line in {probe_log}", file=sys.stderr)
        return 1
    n_launch = probe["launches"]

    def per_entry(d: str, name: str) -> tuple[list[float], float]:
        rows = []
        for f in glob.glob(f"{d}/**/*counter_collection.csv", recursive=True):
            rows += [r for r in csv.DictReader(open(f)) if r["Counter_Name"] == name]
        calib = [float(r["Counter_Value"]) * 1024 for r in rows if CALIB_KERNEL in r["Kernel_Name"]]
        if not calib:
            raise ValueError(f"{d}: no calibration dispatches")
        groups = marker_groups(rows, len(probe["entries"]))
        return [sum(float(r["Counter_Value"]) * 1024 for r in g) / n_launch for g in groups], \
            probe["calibration_bytes_in"] / statistics.mean(calib)

    fetch, f_scale = per_entry(fetch_dir, "FETCH_SIZE")
    write, w_scale = per_entry(write_dir, "WRITE_SIZE")
    lines = [
        "# HBM traffic per op: every timed entry of the bench, FETCH_SIZE + WRITE_SIZE",
        "",
        "Commands (on the MI355X box, fresh autotune cache: the configs are the shipped table's; one",
        "counter per run, each run a separate process):",
        "",
        "```",
        "cd /tmp && export TMPDIR=/tmp && R=<repo root>",
        "timeout -s KILL 300 rocprofv3 --pmc FETCH_SIZE --output-format csv -d $R/gpurun_out/pmc_entries_fetch -- \\",
        "    python $R/bench.py --entry-probe > $R/gpurun_out/pmc_entries_fetch.log",
        "timeout -s KILL 300 rocprofv3 --pmc WRITE_SIZE --output-format csv -d $R/gpurun_out/pmc_entries_write -- \\",
        "    python $R/bench.py --entry-probe > $R/gpurun_out/pmc_entries_write.log",
        "python $R/bench.py --counter-summary $R/gpurun_out/pmc_entries_fetch $R/gpurun_out/pmc_entries_write \\",
        "    $R/gpurun_out/pmc_entries_fetch.log",
        "```",
        "",
        f"`--entry-probe` launches each op {n_launch} times eagerly over the rotating cold copies",
        "between marker kernels, then the calibration kernel `torch.neg` on a 256 MiB fp32 tensor",
        "(256 MiB read, 256 MiB written) 4 times. Counters are KiB per dispatch; an op's bytes are",
        "the sum over its kernels (a split-K GEMM's partials round trip through its reduce shows",
        "here), per launch; scale = known / counted bytes of the calibration kernel:",
        f"FETCH_SIZE x {f_scale:.4f}, WRITE_SIZE x {w_scale:.4f}. Algorithmic bytes: micro.py:82-86 for",
        "the linears (weights, scales, zero points, x, y), x + gamma + codes + scales for the norm,",
        "qweight in + out for the repack.",
        "",
        "| op | config | FETCH bytes | WRITE bytes | traffic / launch | algorithmic | x algorithmic |",
        "|---|---|---:|---:|---:|---:|---:|",
    ]
    for e, fb, wb in zip(probe["entries"], fetch, write):
        fb, wb = fb * f_scale, wb * w_scale
        t = fb + wb
        lines.append(f"| {e['entry']} | {_cfg_name(e.get('config'))} | {fb:.0f} | {wb:.0f} | {t:.0f} | "
                     f"{e['bytes']} | {t / e['bytes']:.3f} |")
    ENTRY_TRAFFIC_SUMMARY.write_text("\n".join(lines) + "\n")
    print(f"wrote {ENTRY_TRAFFIC_SUMMARY} ({len(probe['entries'])} ops)")
    return 0


def _weight_bytes(entry: str) -> int | None:
    """Packed int4 weight bytes (N·K/2) of an entry named after a layer, None otherwise."""
    for name, n, k in SHAPES:
        if entry.startswith(name + " "):
            return n * k // 2
    return None


def instr_summary(pmc_dir: str, probe_log: str) -> int:
    """Write ``INSTR_SUMMARY`` from one ``rocprofv3 --pmc`` run of ``--entry-probe`` with
    ``INSTR_COUNTERS``: per op, the wave instructions it issues by kind (summed over its
    kernels and over the GPU, per launch), per wave, and for the linears per packed weight word
    (8 int4 values), next to the kernel cycles."""
    import csv
    import glob

    probe = _probe_line(probe_log, "entry_probe")
    if probe is None:
        print(f"no entry_probe line in {probe_log}", file=sys.stderr)
        return 1
    n_launch = probe["launches"]
    rows = []
    for f in glob.glob(f"{pmc_dir}/**/*counter_collection.csv", recursive=True):
        rows += list(csv.DictReader(open(f)))
    groups = marker_groups(rows, len(probe["entries"]))
    lines = [
        "# Instruction mix per op: every timed entry of the bench (SQ instruction counters)",
        "",
        "Command (on the MI355X box, fresh autotune cache: the configs are the shipped table's):",
        "",
        "```",
        "cd /tmp && export TMPDIR=/tmp && R=<repo root>",
        f"timeout -s KILL 300 rocprofv3 --pmc {' '.join(INSTR_COUNTERS)} --output-format csv \\",
        "    -d $R/gpurun_out/pmc_entries_instr -- python $R/bench.py --entry-probe > $R/gpurun_out/pmc_entries_instr.log",
        "python $R/bench.py --instr-summary $R/gpurun_out/pmc_entries_instr $R/gpurun_out/pmc_entries_instr.log",
        "```",
        "",
        f"`--entry-probe` launches each op {n_launch} times eagerly between marker kernels. Counts are",
        "wave instructions summed over the GPU and over the op's kernels, per launch. For the linears,",
        "\"VALU per word\" is the lane operations (wave instructions x 64 lanes) per packed weight word",
        "of the layer (N·K/8 int32 words, 8 int4 values each). The exact dequantization of one word",
        "is 13 lane operations (four mask-and-merges into fp16 magic numbers, one shift, four packed",
        "subtractions of the zero point, four packed multiplies by the scale), so a figure near 13",
        "means little other arithmetic; above it, the rest of the kernel's VALU work (or, where M",
        "rows of x are tiled, the same word dequantized by several workgroups). \"MFMA per 64",
        "words\" counts the matrix instructions that consume each 64 words (one 16x16x32 or 32x32x16",
        "B operand). Kernel cycles: GRBM_GUI_ACTIVE per XCD.",
        "",
        "| op | waves | VALU | MFMA | LDS | VMEM rd | SALU | VALU / wave | VALU per word | MFMA per 64 words | cycles |",
        "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|",
    ]
    for e, g in zip(probe["entries"], groups):
        tot = {c: 0.0 for c in INSTR_COUNTERS}
        for r in g:
            if r["Counter_Name"] in tot:
                tot[r["Counter_Name"]] += float(r["Counter_Value"])
        per = {c: v / n_launch for c, v in tot.items()}
        waves = max(per["SQ_WAVES"], 1.0)
        wb = _weight_bytes(e["entry"])
        words = wb / 4 if wb else None
        vw = f"{per['SQ_INSTS_VALU'] * 64 / words:.1f}" if words else "-"
        mw = f"{per['SQ_INSTS_MFMA'] * 64 / words:.2f}" if words else "-"
        lines.append(f"| {e['entry']} | {per['SQ_WAVES']:.0f} | {per['SQ_INSTS_VALU']:.0f} | {per['SQ_INSTS_MFMA']:.0f} | "
                     f"{per['SQ_INSTS_LDS']:.0f} | {per['SQ_INSTS_VMEM_RD']:.0f} | {per['SQ_INSTS_SALU']:.0f} | "
                     f"{per['SQ_INSTS_VALU'] / waves:.0f} | {vw} | {mw} | {per['GRBM_GUI_ACTIVE'] / NUM_XCDS:.0f} |")
    INSTR_SUMMARY.write_text("\n".join(lines) + "\n")
    print(f"wrote {INSTR_SUMMARY} ({len(probe['entries'])} ops)")
    return 0


def _probe_line(log: str, key: str) -> dict | None:  # type: ignore[type-arg]
    for line in Path(log).read_text().splitlines():
        if line.startswith('{"' + key + '"'):
            return json.loads(line)[key]
    return None


def mfma_summary(pmc_dir: str, probe_log: str, timing_log: str) -> int:
    """Write ``MFMA_SUMMARY`` from one ``rocprofv3 --pmc`` run of ``--mfma-probe`` (its log is
    ``probe_log``) and one plain run of it (``timing_log``: the profiler slows graph replays, so
    the event timing comes from a run without it): per GEMM launch, SQ_VALU_MFMA_BUSY_CYCLES
    (summed over every SIMD) over the kernel's cycles (GRBM_GUI_ACTIVE, counted once per XCD)
    times the SIMD count, next to the fraction of the 2.5 PFLOP/s fp16 dense peak."""
    import csv
    import glob

    probe, timing = _probe_line(probe_log, "mfma_probe"), _probe_line(timing_log, "mfma_probe")
    if probe is None or timing is None:
        print(f"no mfma_probe line in {probe_log} or {timing_log}", file=sys.stderr)
        return 1
    if [r["config"] for r in probe["runs"]] != [r["config"] for r in timing["runs"]]:
        raise ValueError("the counter run and the timing run used different configs")
    per: dict = {}  # type: ignore[type-arg]
    for f in glob.glob(f"{pmc_dir}/**/*counter_collection.csv", recursive=True):
        for r in csv.DictReader(open(f)):
            if "gemm" in r["Kernel_Name"] and "reduce" not in r["Kernel_Name"]:
                per.setdefault(int(r["Dispatch_Id"]), {})[r["Counter_Name"]] = float(r["Counter_Value"])
    ids = sorted(per)
    n_launch = probe["launches"]
    # The probe's eager launches come first (layer by layer); later GEMM dispatches belong to
    # its graph timing.
    if len(ids) < n_launch * len(probe["runs"]):
        raise ValueError(f"{pmc_dir}: {len(ids)} GEMM dispatches, expected >= {n_launch * len(probe['runs'])}")
    ids = ids[: n_launch * len(probe["runs"])]
    lines = [
        "# MFMA utilisation and LDS counters of the prefill GEMMs at M=256 (fp16 W4A16 and fp8 W4A8)",
        "",
        "Commands (on the MI355X box, fresh autotune cache: the configs are the shipped table's):",
        "",
        "```",
        "cd /tmp && export TMPDIR=/tmp && R=<repo root>",
        f"timeout -s KILL 150 rocprofv3 --pmc {' '.join(MFMA_COUNTERS)} --output-format csv \\",
        "    -d $R/gpurun_out/pmc_mfma -- python $R/bench.py --mfma-probe > $R/gpurun_out/pmc_mfma.log",
        "python $R/bench.py --mfma-probe > $R/gpurun_out/mfma_timing.log",
        "python $R/bench.py --mfma-summary $R/gpurun_out/pmc_mfma $R/gpurun_out/pmc_mfma.log \\",
        "    $R/gpurun_out/mfma_timing.log",
        "```",
        "",
        f"`--mfma-probe` launches each M=256 GEMM (the fp16 GEMM of gate_up and down at the shipped",
        f"configs, then the W4A8 fp8 GEMM of both at `fp8_gemm_config`) {n_launch} times over",
        "rotating cold weight copies (counters, eager) and times the same launches from a HIP graph",
        "(events, taken from the run without the profiler).",
        f"MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / {NUM_XCDS} XCDs x {NUM_SIMDS} SIMDs): the",
        "share of the kernel's cycles in which an average SIMD's matrix core is busy. The split-K",
        "reduce kernel of down runs no MFMA and is not counted. Rows: mean over the launches.",
        "",
        "LDS bank conflicts = SQ_LDS_BANK_CONFLICT / SQ_INSTS_LDS: cycles lost to bank conflicts per",
        "LDS instruction.",
        "",
        "| layer | GEMM | config | MFMA busy (counters) | us / launch (events) | TFLOP/s | of its dense peak | conflict cycles / LDS instr |",
        "|---|---|---|---:|---:|---:|---:|---:|",
    ]
    for j, run in enumerate(timing["runs"]):
        vals = [per[d] for d in ids[j * n_launch:(j + 1) * n_launch]]
        busy = statistics.mean(v["SQ_VALU_MFMA_BUSY_CYCLES"] / (v["GRBM_GUI_ACTIVE"] / NUM_XCDS * NUM_SIMDS) for v in vals)
        conflict = statistics.mean(v.get("SQ_LDS_BANK_CONFLICT", 0.0) / max(v.get("SQ_INSTS_LDS", 0.0), 1.0)
                                   for v in vals)
        c = run["config"]
        name = f"{c['kernel']} bm{c['block_m']} bn{c['block_n']} bk{c['block_k']} sk{c['split_k']} w{c['num_warps']} st{c['num_stages']}"
        fp8 = run.get("precision") == "fp8"
        peak = FP8_MFMA_PEAK_TFLOPS if fp8 else FP16_MFMA_PEAK_TFLOPS
        lines.append(f"| {run['layer']} | {'W4A8 fp8' if fp8 else 'W4A16 fp16'} | {name} | {100 * busy:.1f}% | "
                     f"{run['us']:.2f} | {run['tflops']:.1f} | {100 * run['tflops'] / peak:.1f}% of "
                     f"{peak / 1000:.1f} PF | {conflict:.2f} |")
    lines += ["", "Raw counters per launch (mean):", "", "| layer | " + " | ".join(MFMA_COUNTERS) + " |",
              "|---|" + "---:|" * len(MFMA_COUNTERS)]
    for j, run in enumerate(probe["runs"]):
        vals = [per[d] for d in ids[j * n_launch:(j + 1) * n_launch]]
        lines.append(f"| {run['layer']} | " + " | ".join(f"{statistics.mean(v[c] for v in vals):.0f}" for c in MFMA_COUNTERS) + " |")
    MFMA_SUMMARY.write_text("\n".join(lines) + "\n")
    print(f"wrote {MFMA_SUMMARY}")
    return 0


PROBE_SUMMARY = ROOT / "profiles" / "gemv_m1_memory_floors.md"


def probe_summary(probe_log: str) -> int:
    """Write ``PROBE_SUMMARY`` from the ``{"read_probe": ...}`` line of a ``--probe`` run: per
    decode shape, the GEMV on the config in use and on the best candidate next to the fastest
    pure-read kernel of each access pattern (the floor the memory system sets for it), and the
    fixed cost of one launch inside a graph."""
    rows = _probe_line(probe_log, "read_probe")
    if rows is None:
        print(f"no read_probe line in {probe_log}", file=sys.stderr)
        return 1
    lines = [
        "# Memory floors of the M=1 decode GEMV (pure-read probes next to the GEMV)",
        "",
        "Command (on the MI355X box, fresh autotune cache: the GEMV configs are the shipped table's):",
        "",
        "```",
        "cd /tmp && export TMPDIR=/tmp && R=<repo root>",
        "python $R/bench.py --probe > $R/gpurun_out/probe.log",
        "python $R/bench.py --probe-summary $R/gpurun_out/probe.log",
        "```",
        "",
        "Every figure is the median over 5 replays of a HIP graph of launches rotating over the",
        "bench's cold layer copies (HIP events on the replay stream), in us per launch. The probes",
        "(bench_probes/read_probes.hip, a library of their own) read with the GEMV's grid",
        "and 128-bit buffer loads and do no arithmetic:",
        "",
        "* tile: the gfx950 tile layout, one workgroup per 16-row tile, its waves splitting the",
        "  tile's 128-wide K steps, each wave step one contiguous 1 KB;",
        "* tile+meta: as tile, plus the step's scale and zero-point words (the GEMV's three loads);",
        "* rows: the TokenForge row-major layout, 16 runs of 64 bytes per load instruction;",
        "* stream: a plain grid-stride read of the weights;",
        "* wave / group / grid: the weights as the tile layout's linear sequence of 1 KB step blocks,",
        "  with each block's scale and zero words (all three loads of a GEMV step), on resident",
        "  grids (256 x 1, 2 or 4 workgroups of 4, 8 or 16 waves, ring depth 2 or 4): every wave",
        "  streaming its own contiguous range (wave), each workgroup owning a contiguous range that",
        "  its waves take round robin (group: the stream form's pattern), or the whole grid taking",
        "  the blocks round robin (grid).",
        "",
        "Best over waves in {1, 2, 4, 8, 16} x ring depth in {2, 4, 8} (stream: grid in {512 .. 4096}).",
        "GB/s are weight bytes (tile+meta, wave, group, grid: plus scales and zeros) per second; the",
        "GEMV's are its algorithmic bytes (weights, scales, zeros, x, y) per second. \"K-split GEMV\" is",
        "the fastest candidate of the K-split form (block_k 128), the decode default before the stream",
        "form.",
        "",
    ]
    empty = [r for r in rows if r["probe"] == "empty"]
    lines += ["| launch | us |", "|---|---:|"]
    lines += [f"| empty kernel, grid {r['grid']} | {r['us']:.2f} |" for r in empty]
    lines += ["", "| shape | GEMV in use | best GEMV candidate | K-split GEMV | tile | tile+meta | rows | stream |",
              "|---|---:|---:|---:|---:|---:|---:|---:|"]
    pats = ("tile", "tile+meta", "rows", "stream")
    for name, n, k in SHAPES:
        mine = [r for r in rows if r.get("layer") == name]
        gemv = [r for r in mine if r["probe"] == "gemv"]
        used = next(r for r in gemv if r["tuned"])
        best = min(gemv, key=lambda r: r["us"])
        ksplit = min((r for r in gemv if r["config"]["block_k"] == 128), key=lambda r: r["us"])
        floor = {p: min((r for r in mine if r["probe"] == p), key=lambda r: r["us"]) for p in pats}
        cell = lambda r: f"{r['us']:.2f} ({r['gbps']:.0f} GB/s)"  # noqa: E731
        lines.append(f"| {name} {n}x{k} | {cell(used)} | {cell(best)} | {cell(ksplit)} | " +
                     " | ".join(cell(floor[p]) for p in pats) + " |")
    lines += ["", "Which blocks are in flight together (weights + scales + zeros, best over the resident grids):", "",
              "| shape | wave | group | grid | GEMV in use / group |", "|---|---:|---:|---:|---:|"]
    for name, n, k in SHAPES:
        mine = [r for r in rows if r.get("layer") == name]
        used = next(r for r in mine if r["probe"] == "gemv" and r["tuned"])
        fl = {p: min((r for r in mine if r["probe"] == p), key=lambda r: r["us"]) for p in ("wave", "group", "grid")}
        cell = lambda r: f"{r['us']:.2f} ({r['gbps']:.0f} GB/s)"  # noqa: E731
        lines.append(f"| {name} {n}x{k} | " + " | ".join(cell(fl[p]) for p in ("wave", "group", "grid")) +
                     f" | {used['us'] / fl['group']['us']:.2f} |")
    lines += ["", "Configs (GEMV in use, best candidate) and probe shapes (waves, depth):", ""]
    for name, n, k in SHAPES:
        mine = [r for r in rows if r.get("layer") == name]
        gemv = [r for r in mine if r["probe"] == "gemv"]
        used = next(r for r in gemv if r["tuned"])
        best = min(gemv, key=lambda r: r["us"])
        fl = {p: min((r for r in mine if r["probe"] == p), key=lambda r: r["us"]) for p in ("tile", "tile+meta", "rows", "stream")}
        fb = {p: min((r for r in mine if r["probe"] == p), key=lambda r: r["us"]) for p in ("wave", "group", "grid")}
        lines.append(f"* {name}: in use `{json.dumps(used['config'])}`; best `{json.dumps(best['config'])}`; " +
                     ", ".join(f"{p} w{fl[p]['waves']} d{fl[p]['depth']}" for p in ("tile", "tile+meta", "rows")) +
                     f", stream grid {fl['stream']['waves']}; " +
                     ", ".join(f"{p} grid {fb[p]['grid']} w{fb[p]['waves']} d{fb[p]['depth']}" for p in ("wave", "group", "grid")))
    PROBE_SUMMARY.write_text("\n".join(lines) + "\n")
    print(f"wrote {PROBE_SUMMARY}")
    return 0


def bytes_moved(m: int, n: int, k: int, group: int = GROUP) -> int:
    """Algorithmic bytes of one W4A16 call (micro.py:82-86)."""
    return n * k // 2 + (k // group) * n * 2 + (k // group) * n // 2 + m * k * 2 + m * n * 2


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _git(*args: str) -> str | None:
    import subprocess

    try:
        out = subprocess.run(["git", *args], cwd=ROOT, check=True, capture_output=True, text=True, timeout=20)
    except (OSError, subprocess.SubprocessError):
        return None
    return out.stdout.strip()


def code_tree_hash() -> str:
    """sha256 over the path and content of every source file under ``CODE_PATHS`` (sorted):
    the same value wherever the tree is, including a copy without ``.git``."""
    import hashlib

    h = hashlib.sha256()
    files = []
    for top in CODE_PATHS:
        p = ROOT / top
        files += [p] if p.is_file() else [f for f in p.rglob("*") if f.is_file() and f.suffix in CODE_SUFFIXES
                                          and "__pycache__" not in f.parts]
    for f in sorted(files):
        h.update(str(f.relative_to(ROOT)).encode() + b"\0" + f.read_bytes() + b"\0")
    return h.hexdigest()


def fingerprint() -> dict:  # type: ignore[type-arg]
    """Environment of a bench line (env.py:51-85): commit, dirty flag and code-tree hash (the git
    fields are null where the tree has no ``.git``, e.g. a copy on the GPU box; the tree hash
    then ties the line to a commit: ``python bench.py --fingerprint`` in a checkout), software
    versions, the kernel library's ABI and the device."""
    import platform

    fp = {"git_sha": _git("rev-parse", "HEAD"), "code_tree": code_tree_hash(), "python": platform.python_version(),
          "torch": torch.__version__, "hip": torch.version.hip, "host_cpu": cpu_model()}
    status = _git("status", "--porcelain", "--", *CODE_PATHS)
    fp["git_dirty"] = None if status is None else bool(status)
    try:
        from tokenforge.kernels import _lib

        fp["library_abi"] = _lib.ABI_VERSION
    except ImportError:
        fp["library_abi"] = None
    if torch.cuda.is_available():
        props = torch.cuda.get_device_properties(0)
        fp["gpu"] = props.name
        fp["arch"] = getattr(props, "gcnArchName", None)
        fp["cus"] = props.multi_processor_count
    return fp


def timed_rows(result: dict) -> dict[str, float]:  # type: ignore[type-arg]
    """Every timed entry of a bench line as ``impl|layer|m`` -> microseconds (micro.py:133)."""
    rows: dict[str, float] = {}
    for key in ("per_shape", "gemv_m2_m4", "gemv_m8_m32", "gemm_small_m", "gemm_m256", "gemm_m1024_m4096"):
        impl = "hip-cfg4" if key == "gemm_small_m" else "hip"  # M=32 is in gemv_m8_m32 too
        for r in result.get(key) or ():
            rows[f"{impl}|{r['layer']}|{r['m']}"] = r["us"]
    for r in result.get("gemm_w4a8_fp8") or ():
        rows[f"hip-fp8|{r['layer']}|{r['m']}"] = r["us"]
    for r in result.get("rmsnorm_fp8") or ():
        rows[f"hip|rmsnorm_fp8|{r['t']}"] = r["us"]
    for r in result.get("vendor_fp16") or ():
        rows[f"vendor-fp16|{r['layer']}|{r['m']}"] = r["us"]
    for r in result.get("stack") or ():
        rows[f"hip-stack|fused|{r['m']}"] = r["fused"]["ms_per_pass"] * 1e3
    return rows


def regression_check(result: dict, path: Path = BASELINE_FILE) -> dict | None:  # type: ignore[type-arg]
    """Each timed entry against the committed baseline for this GPU (micro.py:140-156): the
    entries more than 5% slower, and the headline value's ratio to the baseline's."""
    if not path.exists():
        return None
    doc = json.loads(path.read_text()).get(result["gpu"])
    if doc is None:
        return {"baseline": path.name, "gpu": result["gpu"], "compared": 0, "note": "no baseline for this GPU"}
    rows = timed_rows(result)
    base = doc["us"]
    slower = [{"entry": key, "us": us, "baseline_us": base[key], "slower_pct": 100 * (us / base[key] - 1)}
              for key, us in sorted(rows.items()) if key in base and us > base[key] * (1 + REGRESSION)]
    return {"baseline": path.name, "baseline_code_tree": doc.get("code_tree"), "baseline_reason": doc.get("reason"),
            "compared": sum(key in base for key in rows), "threshold_pct": 100 * REGRESSION,
            "regressions": slower, "pass": not slower, "value_vs_baseline": result["value"] / doc["value"]}


def update_baseline(result: dict, reason: str, path: Path) -> None:  # type: ignore[type-arg]
    """Write this line's timed entries as the baseline for its GPU (micro.py:170-181)."""
    doc = json.loads(path.read_text()) if path.exists() else {}
    doc[result["gpu"]] = {"reason": reason, "code_tree": result["env"]["code_tree"],
                          "git_sha": result["env"]["git_sha"], "value": result["value"], "us": timed_rows(result)}
    path.write_text(json.dumps(doc, indent=1, sort_keys=True) + "\n")


def prefill_x(m: int, k: int, gen: torch.Generator, dev: torch.device) -> torch.Tensor:
    """configs[3]'s activations: fp16 ~N(0, 1) with 1% of the rows (at least one) scaled by 10."""
    x = torch.randn((m, k), generator=gen, device=dev)
    rows = torch.randperm(m, generator=gen, device=dev)[: max(1, m // 100)]
    x[rows] *= 10
    return x.to(torch.float16)


def make_layer(n: int, k: int, dev: torch.device, seed: int):  # type: ignore[no-untyped-def]
    """AWQ-format synthetic layer converted with the GPU repack -> (qweight_t, scales, qzeros)."""
    from tokenforge.kernels.pack import pack_awq, pack_int4

    gen = torch.Generator(device=dev).manual_seed(seed)
    intweight = torch.randint(0, 16, (k, n), generator=gen, device=dev, dtype=torch.int32)
    qweight = pack_int4(intweight)
    del intweight
    zeros = torch.randint(0, 16, (k // GROUP, n), generator=gen, device=dev, dtype=torch.int32)
    scales = (torch.rand((k // GROUP, n), generator=gen, device=dev) * 9e-3 + 1e-3).to(torch.float16)
    w = pack_awq(qweight, pack_int4(zeros), scales, GROUP)
    return w.qweight_t, w.scales, w.qzeros, qweight


def capture(fns: list, warm: int = 4) -> tuple[torch.cuda.CUDAGraph, list]:  # type: ignore[type-arg]
    """Capture ``fns`` (each launches one kernel on the current stream) into one HIP graph."""
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for f in fns[:warm]:
            f()
        stream.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            outs = [f() for f in fns]
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    return graph, outs


def median_replay_ms(graph: torch.cuda.CUDAGraph, launches: int, replays: int = 5) -> float:
    """Median over ``replays`` replays of the per-launch milliseconds of a graph of ``launches``
    launches (one untimed replay first)."""
    time_graph(graph)
    return statistics.median(time_graph(graph) / launches for _ in range(replays))


def time_graph(graph: torch.cuda.CUDAGraph, reps: int = 1) -> float:
    """Milliseconds of ``reps`` replays, HIP events on the replay stream, synced both sides."""
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return float(start.elapsed_time(end))


def rmsnorm_bench(dev: torch.device) -> tuple[list[dict], torch.Tensor]:  # type: ignore[type-arg]
    """fused RMSNorm + FP8 at H=3584 over rotating cold inputs, per T; returns the
    rows and gamma."""
    from tokenforge.kernels.hip.rmsnorm_fp8 import rmsnorm_fp8_quant

    h = NORM_H
    gen = torch.Generator(device="cpu").manual_seed(0)
    outliers = torch.randperm(h, generator=gen)[:8].to(dev)
    gamma = (1 + 0.1 * torch.randn(h, generator=gen)).to(torch.float16).to(dev)
    res = []
    for t in NORM_T:
        copies = max(2, min(64, int(-(-COLD_BYTES // (t * h * 2)))))
        xs = []
        for _ in range(copies):
            x = torch.randn((t, h), device=dev)
            x[:, outliers] *= 20
            xs.append(x.to(torch.float16))
        nbytes = t * h * 2 + h * 2 + t * h + 4 * t
        by_form = {}
        for form in ("auto", "row_per_block", "row_per_wave"):
            g, _ = capture([lambda x=x, form=form: rmsnorm_fp8_quant(x, gamma, 1e-6, None, form=form) for x in xs])
            by_form[form] = median_replay_ms(g, copies) * 1e3
            del g
        us = by_form["auto"]
        gbps = nbytes / (us * 1e-6) / 1e9
        res.append({"t": t, "h": h, "us": us, "gbps": gbps, "frac_hbm": gbps / HBM_PEAK_GBPS,
                    "bytes": nbytes, "us_by_form": by_form})
        log(f"  rmsnorm_fp8   T={t:<5d} {us:8.2f} us {gbps:7.0f} GB/s ({100 * gbps / HBM_PEAK_GBPS:.1f}% of 8 TB/s)"
            f"  [row/block {by_form['row_per_block']:.2f} us, row/wave {by_form['row_per_wave']:.2f} us]")
        del xs
    return res, gamma


def vendor_bench(dev: torch.device, gen: torch.Generator) -> list[dict]:  # type: ignore[type-arg]
    """The vendor's dense fp16 linear beside the library's calls (micro.py:110-114's
    ``cublas-fp16`` impl: ``F.linear(x, W)`` with fp16 weights; on ROCm, hipBLASLt). Each of
    the four shapes at M in {1, 8, 32} (the l4 suite), gate_up and down also at the prefill M;
    the weights rotate over copies of at least 1.1 GB in all, so every launch reads them from
    HBM. GB/s uses the reference's dense byte count (N·K·2 + M·K·2 + M·N·2)."""
    res = []
    for i, (name, n, k) in enumerate(SHAPES):
        copies = max(2, int(-(-COLD_BYTES // (n * k * 2))))
        ws = [(torch.randn((n, k), generator=gen, device=dev) * 0.02).to(torch.float16) for _ in range(copies)]
        for m in (1,) + DECODE_EXTRA_M + (PREFILL_M if i in (2, 3) else ()):
            x = torch.randn((m, k), generator=gen, device=dev).to(torch.float16)
            launches = copies * (2 if m <= 256 else 1)
            g, _ = capture([lambda r=r, x=x: torch.nn.functional.linear(x, ws[r % copies]) for r in range(launches)],
                           warm=2)
            ms = median_replay_ms(g, launches)
            del g
            moved = n * k * 2 + m * k * 2 + m * n * 2
            res.append({"layer": name, "m": m, "n": n, "k": k, "us": ms * 1e3,
                        "gbps": moved / (ms * 1e-3) / 1e9, "tflops": 2 * m * n * k / (ms * 1e-3) / 1e12,
                        "impl": "torch.nn.functional.linear fp16 (hipBLASLt)"})
            log(f"  vendor fp16   {name:13s} M={m:<5d} {ms * 1e3:9.2f} us {moved / (ms * 1e-3) / 1e9:7.0f} GB/s "
                f"{2 * m * n * k / (ms * 1e-3) / 1e12:7.1f} TFLOP/s")
        del ws
        torch.cuda.empty_cache()
    return res


def eager_bench(layers: list, copies: int, xs: list, cfgs: list) -> list[dict]:  # type: ignore[type-arg]
    """The op called eagerly (no graph), as micro.py:67-79 times it: per M=1 call on each shape,
    back to back over the rotating copies. ``us_per_call`` is the stream's time per call (HIP
    events around the loop), ``host_us_per_call`` the Python time to issue one; both for the
    custom op (``torch.ops.tokenforge.w4a16_linear``: dispatch, bucket lookup, metrics, ctypes)
    and for the launcher under it (``w4a16_gemm``: checks and ctypes only)."""
    from tokenforge.kernels.hip.w4a16 import w4a16_gemm

    ops = torch.ops.tokenforge
    res = []
    calls = 40 * copies
    for i, (name, n, k) in enumerate(SHAPES):
        row = {"layer": name, "m": 1}
        for label, fn in (
            ("op", lambda c: ops.w4a16_linear(xs[i], *layers[c][i], None, GROUP, "hip")),
            ("launcher", lambda c: w4a16_gemm(xs[i], *layers[c][i], GROUP, cfgs[i])),
        ):
            for c in range(copies):
                fn(c)
            torch.cuda.synchronize()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            t0 = time.perf_counter()
            for r in range(calls):
                fn(r % copies)
            host_s = time.perf_counter() - t0
            end.record()
            torch.cuda.synchronize()
            row[label] = {"us_per_call": start.elapsed_time(end) * 1e3 / calls, "host_us_per_call": host_s * 1e6 / calls}
        res.append(row)
        log(f"  eager {name:13s} M=1 op {row['op']['us_per_call']:6.2f} us/call (host {row['op']['host_us_per_call']:5.2f}),"
            f" launcher {row['launcher']['us_per_call']:6.2f} us/call (host {row['launcher']['host_us_per_call']:5.2f})")
    return res


STACK_LAYERS = 28
HEAD_DIM = 128
KV_HEADS = 4


def stack_bench(dev: torch.device, gpu: str, ms: tuple[int, ...], tune: bool) -> list[dict]:  # type: ignore[type-arg]
    """tokens/s of one pass through 28 decoder layers, per M (module docstring);
    each M timed with the unfused torch glue, with the fused epilogues (residual adds in
    o_proj and down, SiLU*mul in gate_up; same bits) and with W4A8 qkv and gate_up."""
    from tokenforge.kernels import autotune

    eps = 1e-6
    h = SHAPES[1][1]
    inter = SHAPES[2][1] // 2
    layers = []
    total = 0
    for li in range(STACK_LAYERS):
        ws = [make_layer(n, k, dev, seed=50_000 + 10 * li + i)[:3] for i, (_, n, k) in enumerate(SHAPES)]
        gen = torch.Generator(device=dev).manual_seed(60_000 + li)
        bias = (torch.randn((SHAPES[0][1],), generator=gen, device=dev) * 0.1).to(torch.float16)
        g1 = (1 + 0.1 * torch.randn((h,), generator=gen, device=dev)).to(torch.float16)
        g2 = (1 + 0.1 * torch.randn((h,), generator=gen, device=dev)).to(torch.float16)
        layers.append((ws, bias, g1, g2))
        total += sum(t.numel() * t.element_size() for w in ws for t in w)
    if tune:
        for _, n, k in SHAPES:
            autotune.tune_layer(n, k, GROUP, device=dev, gpu=gpu, buckets=tuple(sorted(set(ms))))
    ops = torch.ops.tokenforge
    q_width = SHAPES[0][1] - 2 * KV_HEADS * HEAD_DIM  # 3584 query columns, then k and v

    def layer_pass(x: torch.Tensor, layer: tuple) -> torch.Tensor:  # type: ignore[type-arg]
        (qkv, o, gu, down), bias, g1, g2 = layer
        m = x.shape[0]
        if mode == "fused":  # norm, fp16(q * scale) and qkv: one kernel at M <= 4, else two
            y = ops.rmsnorm_fp8_w4a16_linear(x, g1, eps, *qkv, bias, GROUP, "hip", "none")
        else:
            q8, s = ops.rmsnorm_fp8_quant(x, g1, eps, None)
            if mode == "w4a8":
                y = ops.w4a8_linear(q8, s, *qkv, bias, GROUP, "hip")
            else:
                a = (q8.to(torch.float32) * s).to(torch.float16)
                y = ops.w4a16_linear(a, *qkv, bias, GROUP, "hip")
        v = y[:, q_width + KV_HEADS * HEAD_DIM:].reshape(m, KV_HEADS, 1, HEAD_DIM)
        attn = v.expand(m, KV_HEADS, h // (KV_HEADS * HEAD_DIM), HEAD_DIM).reshape(m, h)
        if mode == "unfused":
            x = x + ops.w4a16_linear(attn, *o, None, GROUP, "hip")
        else:
            x = ops.w4a16_linear_residual(attn, *o, None, x, GROUP, "hip")
        if mode == "fused":
            act = ops.rmsnorm_fp8_w4a16_linear(x, g2, eps, *gu, None, GROUP, "hip", "silu_mul")
            return ops.w4a16_linear_residual(act, *down, None, x, GROUP, "hip")
        q8, s = ops.rmsnorm_fp8_quant(x, g2, eps, None)
        if mode == "w4a8":
            act = ops.w4a8_linear(q8, s, *gu, None, GROUP, "hip", "silu_mul")
            return ops.w4a16_linear_residual(act, *down, None, x, GROUP, "hip")
        a = (q8.to(torch.float32) * s).to(torch.float16)
        if mode == "unfused":
            y = ops.w4a16_linear(a, *gu, None, GROUP, "hip")
            act = torch.nn.functional.silu(y[:, :inter]) * y[:, inter:]
            return x + ops.w4a16_linear(act, *down, None, GROUP, "hip")
        act = ops.w4a16_linear_silu_mul(a, *gu, None, GROUP, "hip")
        return ops.w4a16_linear_residual(act, *down, None, x, GROUP, "hip")

    res = []
    gen = torch.Generator(device=dev).manual_seed(11)
    mode = "unfused"
    for m in ms:
        x0 = torch.randn((m, h), generator=gen, device=dev).to(torch.float16)

        def full_pass(x0: torch.Tensor = x0) -> torch.Tensor:
            x = x0
            for layer in layers:
                x = layer_pass(x, layer)
            return x

        row: dict = {"m": m, "layers": STACK_LAYERS, "weight_bytes": total}  # type: ignore[type-arg]
        outs_by_mode = {}
        for mode in ("unfused", "fused", "w4a8"):
            g, outs = capture([full_pass], warm=1)
            ms_pass = median_replay_ms(g, 1)  # replays the graph: outs[0] holds the pass's output
            if not bool(torch.isfinite(outs[0]).all()):
                raise RuntimeError(f"stack pass at M={m} produced non-finite values")
            outs_by_mode[mode] = outs[0]
            step_bytes = sum(bytes_moved(m, n, k) for _, n, k in SHAPES) * STACK_LAYERS
            flops = 2 * m * sum(n * k for _, n, k in SHAPES) * STACK_LAYERS
            key = mode
            row[key] = {"ms_per_pass": ms_pass, "tokens_per_s": m / (ms_pass * 1e-3),
                        "linear_gbps": step_bytes / (ms_pass * 1e-3) / 1e9,
                        "linear_tflops": flops / (ms_pass * 1e-3) / 1e12}
            log(f"  stack M={m:<5d} {key:8s} {ms_pass * 1e3:9.1f} us/pass {m / (ms_pass * 1e-3):9.0f} tok/s "
                f"({step_bytes / (ms_pass * 1e-3) / 1e9:.0f} GB/s of linear bytes)")
            del g, outs
        row["fused_equals_unfused"] = bool(torch.equal(outs_by_mode["unfused"], outs_by_mode["fused"]))
        ref = outs_by_mode["fused"].float()
        row["w4a8_normwise_vs_fp16_input"] = float((outs_by_mode["w4a8"].float() - ref).abs().max() / ref.abs().max())
        row["tokens_per_s"] = row["fused"]["tokens_per_s"]
        res.append(row)
        del outs_by_mode
    del layers
    torch.cuda.empty_cache()
    return res


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or the platform's processor string."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def _median_s(fn, runs: int, budget_s: float) -> tuple[float, int]:  # type: ignore[no-untyped-def]
    """Median seconds of ``fn`` over up to ``runs`` runs within about ``budget_s`` (one warmup)."""
    fn()
    times: list[float] = []
    t_end = time.perf_counter() + budget_s
    while len(times) < runs and (not times or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baselines(layers_tf: list, gate_awq: torch.Tensor, norm_gamma: torch.Tensor,  # type: ignore[type-arg]
                  budget_s: float = 12.0) -> dict:  # type: ignore[type-arg]
    """reference.py's CPU path restated in torch on the host cores (oracle/cpu_path.py), on
    bounded samples of the benchmarked work: the M=1 decode step (the headline baseline), the
    M=256 GEMM of gate_up and down, the fused RMSNorm + FP8 at T=4096 and the AWQ -> TokenForge
    repack of gate_up, and beside the added rows the M=8 decode step and the M=16 GEMMs.
    ``layers_tf``: the four linears in the TokenForge layout on the host."""
    from oracle.cpu_path import repack_awq_to_tf_cpu, rmsnorm_fp8_torch_cpu, w4a16_torch_cpu

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    model = cpu_model()
    gen = torch.Generator().manual_seed(3)
    xs = [torch.randn((1, k), generator=gen).half() for _, _, k in SHAPES]

    def step() -> None:
        for (qw, sc, qz), x in zip(layers_tf, xs):
            w4a16_torch_cpu(x, qw, sc, qz, GROUP)

    med, runs = _median_s(step, 20, budget_s)
    step_bytes = sum(bytes_moved(1, n, k) for _, n, k in SHAPES)
    out = {
        "value": step_bytes / med / 1e9,
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "cpu_model": model,
        "sample": f"one M=1 decode step over the 4 Qwen2.5-7B linears (dequantize per call + fp32 "
                  f"matmul, reference.py:24-32 in torch), median of {runs} runs, {med * 1e3:.0f} ms/step",
        "ms_per_step": med * 1e3,
    }
    xs8 = [torch.randn((8, k), generator=gen).half() for _, _, k in SHAPES]

    def step8() -> None:
        for (qw, sc, qz), x in zip(layers_tf, xs8):
            w4a16_torch_cpu(x, qw, sc, qz, GROUP)

    med, runs = _median_s(step8, 3, budget_s / 4)
    decode_m8 = {"gbps": sum(bytes_moved(8, n, k) for _, n, k in SHAPES) / med / 1e9, "ms_per_step": med * 1e3,
                 "runs": runs, "sample": "one M=8 step over the 4 linears"}
    gemm = {}
    gemm16 = {}
    for i in (2, 3):
        name, n, k = SHAPES[i]
        qw, sc, qz = layers_tf[i]
        for m, table, runs_max in ((256, gemm, 3), (16, gemm16, 2)):
            x = torch.randn((m, k), generator=gen).half()
            med, runs = _median_s(lambda x=x: w4a16_torch_cpu(x, qw, sc, qz, GROUP), runs_max, budget_s / 4)
            table[name] = {"tflops": 2 * m * n * k / med / 1e12, "ms": med * 1e3, "runs": runs}
    t = NORM_T[-1]
    x = torch.randn((t, NORM_H), generator=gen)
    x[:, torch.randperm(NORM_H, generator=gen)[:8]] *= 20
    x = x.half()
    med, runs = _median_s(lambda: rmsnorm_fp8_torch_cpu(x, norm_gamma, 1e-6), 10, budget_s / 4)
    nbytes = t * NORM_H * 2 + NORM_H * 2 + t * NORM_H + 4 * t
    norm = {"t": t, "gbps": nbytes / med / 1e9, "us": med * 1e6, "runs": runs}
    med, runs = _median_s(lambda: repack_awq_to_tf_cpu(gate_awq), 3, budget_s / 2)
    n, k = SHAPES[2][1], SHAPES[2][2]
    repack = {"gvalues_per_s": n * k / med / 1e9, "gbps": n * k / med / 1e9, "ms": med * 1e3, "runs": runs}
    common = {"cores": out["cores"], "kind": "port", "cpu_model": model}
    return {"decode": out, "gemm_m256": {kk: dict(v, **common) for kk, v in gemm.items()},
            "gemm_m16": {kk: dict(v, **common) for kk, v in gemm16.items()}, "decode_m8": dict(decode_m8, **common),
            "rmsnorm_t4096": dict(norm, **common), "repack_gate_up": dict(repack, **common)}


def read_probes(dev: torch.device, layers: list, copies: int, xs: list, cfgs: list) -> int:  # type: ignore[type-arg]
    """--probe: pure-read kernels with the decode GEMV's grid and access patterns (no arithmetic)
    on the same rotating cold copies, against the GEMV itself, plus the fixed cost of a launch.
    Prints a table to stderr and one JSON line {"read_probe": ...} to stdout."""
    import ctypes

    from tokenforge.kernels.config import candidate_configs
    from tokenforge.kernels.hip.w4a16 import w4a16_gemm

    plib = ctypes.CDLL(str(ROOT / "bench_probes" / "lib" / "libtokenforge_read_probes.so"))
    p_, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
    plib.tfp_read.argtypes = [i32, p_, p_, p_, i64, i64, i32, i32, p_, p_]
    plib.tfp_out_words.argtypes = [i64, i32]
    plib.tfp_out_words.restype = i64
    plib.tfp_empty.argtypes = [i32, p_]
    plib.tfp_read_blocks.argtypes = [i32, p_, p_, p_, i64, i64, i32, i32, i32, p_, p_]
    stream = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    rows = []

    for grid in (256, 2368):
        g, _ = capture([lambda grid=grid: plib.tfp_empty(grid, stream())] * 200)
        us = median_replay_ms(g, 200) * 1e3
        rows.append({"probe": "empty", "grid": grid, "us": us})
        log(f"  empty kernel grid {grid:5d}: {us:.2f} us per launch")
        del g
    names = {0: "tile", 1: "tile+meta", 2: "rows", 3: "stream"}
    for i, (name, n, k) in enumerate(SHAPES):
        weight_bytes = n * k // 2
        meta_bytes = (k // GROUP) * n * 2 + (k // GROUP) * n // 2
        x = xs[i]
        sweep = []
        for cfg in [cfgs[i]] + [c for c in candidate_configs(1, GROUP) if c != cfgs[i]]:
            g, _ = capture([lambda c=c, cfg=cfg: w4a16_gemm(x, *layers[c][i], GROUP, cfg) for c in range(copies)])
            us = median_replay_ms(g, copies) * 1e3
            del g
            sweep.append((us, cfg))
            rows.append({"probe": "gemv", "layer": name, "n": n, "k": k, "config": cfg.to_dict(), "us": us,
                         "gbps": bytes_moved(1, n, k) / us / 1e3, "tuned": cfg == cfgs[i]})
        for us, cfg in [sweep[0]] + sorted(sweep[1:], key=lambda t: t[0])[:4]:
            log(f"  {name:13s} GEMV {'tuned' if cfg == cfgs[i] else 'cand '} bm{cfg.block_m} bn{cfg.block_n} "
                f"bk{cfg.block_k} w{cfg.num_warps} st{cfg.num_stages}: {us:6.2f} us "
                f"{bytes_moved(1, n, k) / us / 1e3:6.0f} GB/s")
        best: dict[int, tuple[float, int, int]] = {}
        for pattern in (0, 1, 2, 3):
            combos = [(w, d) for w in (1, 2, 4, 8, 16) for d in (2, 4, 8)] if pattern < 3 else \
                [(g_, 0) for g_ in (512, 1024, 2048, 4096)]
            for waves, depth in combos:
                words = plib.tfp_out_words(n, waves) if pattern < 3 else waves * 256
                out = torch.empty(words, dtype=torch.int32, device=dev)
                fns = [lambda c=c, waves=waves, depth=depth, pattern=pattern, out=out: plib.tfp_read(
                    pattern, layers[c][i][0].data_ptr(), layers[c][i][1].data_ptr(), layers[c][i][2].data_ptr(),
                    n, k, waves, depth, out.data_ptr(), stream()) for c in range(copies)]
                assert fns[0]() == 0, (pattern, waves, depth)
                g, _ = capture(fns)
                us = median_replay_ms(g, copies) * 1e3
                del g
                nbytes = weight_bytes + (meta_bytes if pattern == 1 else 0)
                rows.append({"probe": names[pattern], "layer": name, "n": n, "k": k, "waves": waves,
                             "depth": depth, "us": us, "gbps": nbytes / us / 1e3})
                if pattern not in best or us < best[pattern][0]:
                    best[pattern] = (us, waves, depth)
        for pattern, (us, waves, depth) in sorted(best.items()):
            nbytes = weight_bytes + (meta_bytes if pattern == 1 else 0)
            log(f"  {name:13s} {names[pattern]:9s} best {us:6.2f} us {nbytes / us / 1e3:6.0f} GB/s "
                f"(waves {waves}, depth {depth})")
        # The stream form's question: which blocks should be in flight together (patterns 4-6,
        # weights plus scale and zero reads, on resident grids of 256 x per-CU workgroups).
        for pattern, pname in ((4, "wave"), (5, "group"), (6, "grid")):
            top = None
            for waves in (4, 8, 16):
                for per_cu in (1, 2, 4):
                    if waves * per_cu > 32:
                        continue
                    for depth in (2, 4):
                        grid = 256 * per_cu
                        out = torch.empty(grid * waves * 64, dtype=torch.int32, device=dev)
                        fns = [lambda c=c, waves=waves, depth=depth, pattern=pattern, out=out, grid=grid:
                               plib.tfp_read_blocks(pattern, layers[c][i][0].data_ptr(), layers[c][i][1].data_ptr(),
                                                    layers[c][i][2].data_ptr(), n, k, grid, waves, depth,
                                                    out.data_ptr(), stream()) for c in range(copies)]
                        assert fns[0]() == 0, (pattern, grid, waves, depth)
                        g, _ = capture(fns)
                        us = median_replay_ms(g, copies) * 1e3
                        del g
                        gbps = (weight_bytes + meta_bytes) / us / 1e3
                        rows.append({"probe": pname, "layer": name, "n": n, "k": k, "grid": grid, "waves": waves,
                                     "depth": depth, "us": us, "gbps": gbps})
                        if top is None or us < top[0]:
                            top = (us, grid, waves, depth)
            assert top is not None
            log(f"  {name:13s} {pname:9s} best {top[0]:6.2f} us (grid {top[1]}, waves {top[2]}, depth {top[3]})")
    print(json.dumps({"read_probe": rows}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--tune", action="store_true",
                    help="retune every timed shape and bucket into the autotune cache first")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--detail", type=str, default=None, help="write per-shape details as JSON")
    ap.add_argument("--full", action="store_true",
                    help="also sweep the GEMM over M in {16..4096} on cold copies into --detail (gemm_sweep)")
    ap.add_argument("--stack", action="store_true",
                    help="accepted for older command lines: the stack runs at M in {1, 8, 32, 2048} by default")
    ap.add_argument("--no-stack", action="store_true", help="skip the stack (configs[4])")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="eager gate_up GEMV launches + a calibration kernel, for rocprofv3 --pmc")
    ap.add_argument("--traffic-summary", nargs=3, metavar=("FETCH_DIR", "WRITE_DIR", "PROBE_LOG"),
                    help="write the committed traffic summary from two --traffic-probe counter runs")
    ap.add_argument("--mfma-probe", action="store_true",
                    help="eager + graph-timed launches of the tuned M=256 GEMMs, for rocprofv3 --pmc")
    ap.add_argument("--mfma-summary", nargs=3, metavar=("PMC_DIR", "PROBE_LOG", "TIMING_LOG"),
                    help="write the committed MFMA-utilisation summary from a --mfma-probe counter run "
                         "and a plain --mfma-probe run")
    ap.add_argument("--stats-summary", nargs=5,
                    metavar=("PROF_DIR", "BENCH_LOG", "PROF_LOG", "KPROF_DIR", "KPROBE_LOG"),
                    help="write the committed kernel-statistics summary from a rocprofv3 kernel-trace run")
    ap.add_argument("--probe-summary", metavar="PROBE_LOG",
                    help="write the committed memory-floor summary from a --probe run's output")
    ap.add_argument("--entry-probe", action="store_true",
                    help="eager launches of every op the bench line times, between marker kernels, for rocprofv3")
    ap.add_argument("--counter-summary", nargs=3, metavar=("FETCH_DIR", "WRITE_DIR", "PROBE_LOG"),
                    help="write the committed per-op HBM traffic summary from two --entry-probe counter runs")
    ap.add_argument("--instr-summary", nargs=2, metavar=("PMC_DIR", "PROBE_LOG"),
                    help="write the committed per-op instruction-mix summary from an --entry-probe counter run")
    ap.add_argument("--probe", action="store_true",
                    help="memory floors of the GEMV's access patterns (bench_probes/lib/libtokenforge_read_probes.so), "
                         "next to the GEMV itself on the cached or default configs")
    ap.add_argument("--check", action="store_true",
                    help="exit 1 when an entry is more than 5%% slower than the committed baseline")
    ap.add_argument("--update-baseline", metavar="PATH", nargs="?", const=str(BASELINE_FILE), default=None,
                    help="write this run's timed entries as the baseline for its GPU (needs --reason)")
    ap.add_argument("--reason", default="", help="why the baseline changes (with --update-baseline)")
    ap.add_argument("--fingerprint", action="store_true", help="print the environment fingerprint and exit")
    args = ap.parse_args()
    if args.fingerprint:
        print(json.dumps(fingerprint()))
        return 0
    if args.update_baseline is not None and not args.reason:
        print("--update-baseline needs --reason", file=sys.stderr)
        return 2
    if args.stats_summary:
        return stats_summary(*args.stats_summary)
    if args.probe_summary:
        return probe_summary(args.probe_summary)
    if args.traffic_summary:
        return traffic_summary(*args.traffic_summary)
    if args.mfma_summary:
        return mfma_summary(*args.mfma_summary)
    if args.counter_summary:
        return counter_summary(*args.counter_summary)
    if args.instr_summary:
        return instr_summary(*args.instr_summary)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(
            "bench.py measures one GPU: this build's hot path is single-GPU (no collectives); "
            "run with --gpus 1",
            file=sys.stderr,
        )
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X (gfx950) GPU", file=sys.stderr)
        return 1

    import tokenforge.kernels.ops  # noqa: F401
    from tokenforge.kernels import autotune
    from tokenforge.kernels.device import gpu_identity
    from tokenforge.kernels.hip.w4a16 import w4a16_gemm

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gpu = gpu_identity(dev)
    os.environ.setdefault(autotune.CACHE_DIR_ENV, str(ROOT / "gpurun_out" / "autotune"))
    step_bytes = sum(bytes_moved(1, n, k) for _, n, k in SHAPES)
    copies = max(2, int(-(-COLD_BYTES // step_bytes)))

    t0 = time.perf_counter()
    layers = [[make_layer(n, k, dev, seed=1000 * c + i) for i, (_, n, k) in enumerate(SHAPES)] for c in range(copies)]
    # Load-time repack throughput (pack.py:141-143) on the largest weight, for the record.
    from tokenforge.kernels.pack import repack_awq_to_tf

    gate_awq = layers[0][2][3]
    g_rep, _ = capture([lambda: repack_awq_to_tf(gate_awq)] * 8, warm=2)
    rep_ms = median_replay_ms(g_rep, 8)
    del g_rep
    gate_awq_host = None if args.no_cpu else gate_awq.cpu()
    gate_awq_dev = gate_awq if args.entry_probe else None
    del gate_awq
    for c in range(copies):
        layers[c] = [t[:3] for t in layers[c]]
    torch.cuda.synchronize()
    log(f"setup: {copies} layer copies ({copies * step_bytes / 1e9:.2f} GB) in {time.perf_counter() - t0:.1f}s")

    if args.tune:
        t0 = time.perf_counter()
        for _, n, k in SHAPES:
            buckets = (1, 2, 4) + (PREFILL_M if n == 37888 or k == 18944 else ())
            if args.full and (n == 37888 or k == 18944):
                buckets = tuple(sorted(set(buckets) | set(SWEEP_M)))
            autotune.tune_layer(n, k, GROUP, device=dev, gpu=gpu, buckets=buckets)
        log(f"autotune: {time.perf_counter() - t0:.1f}s")

    def config(m: int, n: int, k: int) -> tuple:  # type: ignore[type-arg]
        """(config, where it came from) that the hot path's lookup returns for this call."""
        return autotune.lookup(gpu, m, n, k, GROUP), autotune.config_source(gpu, m, n, k, GROUP)

    cfg1, src1 = zip(*(config(1, n, k) for _, n, k in SHAPES))
    for (name, _, _), c, src in zip(SHAPES, cfg1, src1):
        log(f"config M=1 {name}: {c} ({src})")

    gen = torch.Generator(device=dev).manual_seed(7)
    xs = [torch.randn((1, k), generator=gen, device=dev).to(torch.float16) for _, _, k in SHAPES]

    if args.probe:
        return read_probes(dev, layers, copies, xs, cfg1)

    if args.traffic_probe:
        from tokenforge.kernels.config import candidate_configs, stream_form_applies

        qw_s_z = [layers[c][2] for c in range(copies)]
        _, n_g, k_g = SHAPES[2]
        # the candidates that run on gate_up (a stream form's K split needs a step per wave)
        cands = [c for c in candidate_configs(1, GROUP)
                 if not c.stream or stream_form_applies(1, n_g, k_g, c.num_warps, max_m=c.block_m, split_k=c.split_k)]
        for cfg in cands:
            for c in range(copies):  # cold: each launch reads a copy the previous ones evicted
                qw, sc, qz = qw_s_z[c % copies]
                w4a16_gemm(xs[2], qw, sc, qz, GROUP, cfg)
        src = torch.randn(CALIB_BYTES // 4, device=dev)
        dst = torch.empty_like(src)
        for _ in range(4):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        print(json.dumps({"traffic_probe": {"kernel": "gate_up GEMV M=1", "launches": copies,
                                            "configs": [c.to_dict() for c in cands],
                                            "algorithmic_bytes": bytes_moved(1, n_g, k_g),
                                            "calibration": "torch.neg", "calibration_bytes_in": CALIB_BYTES,
                                            "calibration_bytes_out": CALIB_BYTES}}), flush=True)
        return 0

    def launcher(c: int, i: int, m_x: list, cfgs: list):  # type: ignore[no-untyped-def]
        qw, s, z = layers[c][i]
        x, cfg = m_x[i], cfgs[i]
        return lambda: w4a16_gemm(x, qw, s, z, GROUP, cfg)

    if args.entry_probe:
        # Eager launches of every op the bench line times, each `copies` times over the rotating
        # cold copies, with a marker kernel before each op and the calibration kernel at the end,
        # for rocprofv3 runs (kernel trace, FETCH_SIZE, WRITE_SIZE) that group dispatches by op.
        from tokenforge.kernels.config import fp8_gemm_config
        from tokenforge.kernels.hip.rmsnorm_fp8 import rmsnorm_fp8_quant
        from tokenforge.kernels.hip.w4a16 import w4a8_gemm_ex

        entries: list = []  # type: ignore[type-arg]

        def add(label: dict, fn, nbytes: int) -> None:  # type: ignore[no-untyped-def,type-arg]
            if all(e[0]["entry"] != label["entry"] for e in entries):  # M=32 of gate_up and down: once
                entries.append((dict(label, bytes=nbytes), fn))

        for m in (1, 2, 4) + DECODE_EXTRA_M:
            xm = xs if m == 1 else [torch.randn((m, k), generator=gen, device=dev).to(torch.float16) for _, _, k in SHAPES]
            for i, (name, n, k) in enumerate(SHAPES):
                cfg = config(m, n, k)[0]
                add({"entry": f"{name} M={m}", "config": cfg.to_dict()},
                    lambda c, i=i, xm=xm, cfg=cfg: launcher(c, i, xm, [cfg] * len(SHAPES))(), bytes_moved(m, n, k))
        for m in SMALL_M + PREFILL_M:
            for i in (2, 3):
                name, n, k = SHAPES[i]
                cfg = config(m, n, k)[0]
                xm = [None] * len(SHAPES)
                xm[i] = prefill_x(m, k, gen, dev)
                add({"entry": f"{name} M={m}", "config": cfg.to_dict()},
                    lambda c, i=i, xm=xm, cfg=cfg: launcher(c, i, xm, [cfg] * len(SHAPES))(), bytes_moved(m, n, k))
        for m in PREFILL_M:
            for i in (2, 3):
                name, n, k = SHAPES[i]
                cfg = fp8_gemm_config(m, n, k)
                x8 = (torch.randn((m, k), generator=gen, device=dev) * 50).to(torch.float8_e4m3fn)
                xs8 = torch.rand((m,), generator=gen, device=dev) * 0.01 + 0.001
                add({"entry": f"{name} M={m} W4A8", "config": cfg.to_dict()},
                    lambda c, i=i, x8=x8, xs8=xs8, cfg=cfg: w4a8_gemm_ex(x8, xs8, *layers[c][i], GROUP, cfg),
                    bytes_moved(m, n, k) - m * k + 4 * m)  # e4m3 x (one byte) and its row scales
        gamma = (1 + 0.1 * torch.randn(NORM_H, generator=gen, device=dev)).to(torch.float16)
        for t in NORM_T:
            n_in = max(2, min(64, int(-(-COLD_BYTES // (t * NORM_H * 2)))))
            xin = [torch.randn((t, NORM_H), generator=gen, device=dev).to(torch.float16) for _ in range(n_in)]
            add({"entry": f"rmsnorm_fp8 T={t}"},
                lambda c, xin=xin: rmsnorm_fp8_quant(xin[c % len(xin)], gamma, 1e-6, None),
                t * NORM_H * 2 + NORM_H * 2 + t * NORM_H + 4 * t)
        add({"entry": "repack gate_up_proj"}, lambda c: repack_awq_to_tf(gate_awq_dev),
            SHAPES[2][1] * SHAPES[2][2] // 2 * 2)
        marker = torch.zeros(1, dtype=torch.int32, device=dev)
        src = torch.randn(CALIB_BYTES // 4, device=dev)
        dst = torch.empty_like(src)
        for _, fn in entries:
            torch.bitwise_not(marker, out=marker)
            for c in range(copies):
                fn(c)
            torch.cuda.synchronize()
        torch.bitwise_not(marker, out=marker)
        for _ in range(4):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        print(json.dumps({"entry_probe": {"launches": copies, "entries": [e[0] for e in entries],
                                          "calibration": "torch.neg", "calibration_bytes_in": CALIB_BYTES,
                                          "calibration_bytes_out": CALIB_BYTES}}), flush=True)
        return 0

    if args.mfma_probe:
        # First the eager launches the counters see (each GEMM's in turn: the fp16 GEMM on
        # gate_up and down, then the W4A8 fp8 GEMM on both), then the graph timing of the same
        # launches (its dispatches come after and are not counted).
        from tokenforge.kernels.config import fp8_gemm_config
        from tokenforge.kernels.hip.w4a16 import w4a8_gemm_ex

        m = 256
        gemms = []  # (label, config, fn(c))
        for i in (2, 3):
            name, n, k = SHAPES[i]
            cfg = config(m, n, k)[0]
            xm = [None] * len(SHAPES)
            xm[i] = prefill_x(m, k, gen, dev)
            gemms.append(({"layer": name, "m": m, "n": n, "k": k, "precision": "fp16"}, cfg,
                          lambda c, i=i, xm=xm, cfg=cfg: launcher(c, i, xm, [cfg] * len(SHAPES))()))
        for i in (2, 3):
            name, n, k = SHAPES[i]
            cfg = fp8_gemm_config(m, n, k)
            x8 = (torch.randn((m, k), generator=gen, device=dev) * 50).to(torch.float8_e4m3fn)
            xs8 = torch.rand((m,), generator=gen, device=dev) * 0.01 + 0.001
            gemms.append(({"layer": name, "m": m, "n": n, "k": k, "precision": "fp8"}, cfg,
                          lambda c, i=i, x8=x8, xs8=xs8, cfg=cfg: w4a8_gemm_ex(x8, xs8, *layers[c][i], GROUP, cfg)))
        for _, _, fn in gemms:
            for c in range(MFMA_LAUNCHES):
                fn(c % copies)
        torch.cuda.synchronize()
        runs = []
        for label, cfg, fn in gemms:
            g, _ = capture([lambda r=r, fn=fn: fn(r % copies) for r in range(2 * copies)])
            ms = median_replay_ms(g, 2 * copies)
            runs.append(dict(label, config=cfg.to_dict(), us=ms * 1e3,
                             tflops=2 * m * label["n"] * label["k"] / (ms * 1e-3) / 1e12))
            del g
        print(json.dumps({"mfma_probe": {"launches": MFMA_LAUNCHES, "runs": runs}}), flush=True)
        return 0

    def steps(count: int, offset: int = 0) -> list:  # type: ignore[type-arg]
        fns = []
        for st in range(count):
            c = (offset + st) % copies
            fns += [launcher(c, i, xs, cfg1) for i in range(len(SHAPES))]
        return fns

    warm_graph, _ = capture(steps(max(1, args.warmup)))
    timed_graph, _ = capture(steps(args.steps, offset=args.warmup))
    time_graph(warm_graph)
    elapsed_ms = time_graph(timed_graph)
    value = args.steps * step_bytes / (elapsed_ms * 1e-3) / 1e9
    log(f"decode step: {elapsed_ms / args.steps * 1e3:.1f} us/step, {value:.0f} GB/s")

    # Per-shape average launch duration (graph of launches rotating over the copies).
    per_shape = []
    reps = 4 * copies
    for i, (name, n, k) in enumerate(SHAPES):
        g, _ = capture([launcher(r % copies, i, xs, cfg1) for r in range(reps)])
        ms = median_replay_ms(g, reps)
        gbps = bytes_moved(1, n, k) / (ms * 1e-3) / 1e9
        per_shape.append({"layer": name, "m": 1, "n": n, "k": k, "us": ms * 1e3, "gbps": gbps,
                          "frac_hbm": gbps / HBM_PEAK_GBPS, "config": cfg1[i].to_dict(), "config_source": src1[i]})
        log(f"  {name:13s} M=1 {ms * 1e3:8.2f} us {gbps:7.0f} GB/s ({100 * gbps / HBM_PEAK_GBPS:.1f}% of 8 TB/s)")
    dom = per_shape[2]

    # the GEMV at M = 2 and 4 on the four shapes (M = 1 is per_shape), and the
    # reference's l4 suite's M = 8 and 32 (micro.py:58), with the tuned buckets' configs.
    gemv_m24 = []
    for m in (2, 4) + DECODE_EXTRA_M:
        xm_all = [torch.randn((m, k), generator=gen, device=dev).to(torch.float16) for _, _, k in SHAPES]
        cfgm, srcm = zip(*(config(m, n, k) for _, n, k in SHAPES))
        for i, (name, n, k) in enumerate(SHAPES):
            g, _ = capture([launcher(r % copies, i, xm_all, cfgm) for r in range(reps)])
            ms = median_replay_ms(g, reps)
            gbps = bytes_moved(m, n, k) / (ms * 1e-3) / 1e9
            gemv_m24.append({"layer": name, "m": m, "n": n, "k": k, "us": ms * 1e3, "gbps": gbps,
                             "frac_hbm": gbps / HBM_PEAK_GBPS, "config": cfgm[i].to_dict(),
                             "config_source": srcm[i]})
            log(f"  {name:13s} M={m} {ms * 1e3:8.2f} us {gbps:7.0f} GB/s ({100 * gbps / HBM_PEAK_GBPS:.1f}% of 8 TB/s)")
            del g

    gemv_m8_m32 = [r for r in gemv_m24 if r["m"] in DECODE_EXTRA_M]
    gemv_m24 = [r for r in gemv_m24 if r["m"] not in DECODE_EXTRA_M]

    # the GEMM at M = 16..128 and at the prefill M = 256, 1024 and 4096 on gate_up
    # and down (activations with 1% of the rows scaled by 10).
    gemm = []
    for m in SMALL_M + PREFILL_M:
        for i in (2, 3):
            name, n, k = SHAPES[i]
            cfg, src = config(m, n, k)
            xm = [None] * len(SHAPES)
            xm[i] = prefill_x(m, k, gen, dev)
            launches = 2 * copies if m <= 256 else copies
            g, _ = capture([launcher(r % copies, i, xm, [cfg] * len(SHAPES)) for r in range(launches)])
            ms = median_replay_ms(g, launches)
            del g, xm
            tflops = 2 * m * n * k / (ms * 1e-3) / 1e12
            gemm.append({"layer": name, "m": m, "n": n, "k": k, "us": ms * 1e3, "tflops": tflops,
                         "frac_mfma": tflops / FP16_MFMA_PEAK_TFLOPS, "config": cfg.to_dict(), "config_source": src})
            log(f"  {name:13s} M={m:<4d} {ms * 1e3:8.2f} us {tflops:7.1f} TFLOP/s "
                f"({100 * tflops / FP16_MFMA_PEAK_TFLOPS:.1f}% of 2.5 PF)  {cfg} ({src})")

    # W4A8 prefill on the fp8 matrix cores (the op's choice at these M): e4m3 x with per-row
    # scales, same weights and M as the W4A16 prefill GEMM above.
    from tokenforge.kernels.config import fp8_gemm_config
    from tokenforge.kernels.hip.w4a16 import w4a8_gemm_ex

    gemm8 = []
    for m in PREFILL_M:
        for i in (2, 3):
            name, n, k = SHAPES[i]
            cfg = fp8_gemm_config(m, n, k)
            x8 = (torch.randn((m, k), generator=gen, device=dev) * 50).to(torch.float8_e4m3fn)
            xs8 = torch.rand((m,), generator=gen, device=dev) * 0.01 + 0.001
            launches = 2 * copies if m <= 256 else copies
            g, _ = capture([lambda r=r, x8=x8, xs8=xs8, cfg=cfg, i=i: w4a8_gemm_ex(x8, xs8, *layers[r % copies][i], GROUP, cfg)
                            for r in range(launches)])
            ms = median_replay_ms(g, launches)
            del g, x8
            tflops = 2 * m * n * k / (ms * 1e-3) / 1e12
            gemm8.append({"layer": name, "m": m, "n": n, "k": k, "us": ms * 1e3, "tflops": tflops,
                          "frac_fp16_mfma": tflops / FP16_MFMA_PEAK_TFLOPS, "frac_fp8_mfma": tflops / FP8_MFMA_PEAK_TFLOPS,
                          "config": cfg.to_dict(), "config_source": "fp8_gemm_config"})
            log(f"  {name:13s} M={m:<4d} W4A8 fp8 {ms * 1e3:8.2f} us {tflops:7.1f} TFLOP/s "
                f"({100 * tflops / FP16_MFMA_PEAK_TFLOPS:.1f}% of 2.5 PF fp16, {100 * tflops / FP8_MFMA_PEAK_TFLOPS:.1f}% of 5 PF fp8)  {cfg}")

    norm, norm_gamma = rmsnorm_bench(dev)

    # The box's achievable copy bandwidth (torch's device copy, 1 GiB in and out over 4 launches
    # of 256 MiB), the yardstick next to the 8 TB/s HBM peak.
    src = torch.empty(COPY_BYTES // 2, dtype=torch.float16, device=dev).normal_()
    dst = torch.empty_like(src)
    chunk = src.numel() // 4
    g_copy, _ = capture([lambda i=i: dst[i * chunk:(i + 1) * chunk].copy_(src[i * chunk:(i + 1) * chunk])
                         for i in range(4)], warm=1)
    copy_ms = median_replay_ms(g_copy, 1)
    copy_gbps = 2 * COPY_BYTES / (copy_ms * 1e-3) / 1e9
    log(f"device copy: {copy_gbps:.0f} GB/s (read + write)")
    del g_copy, src, dst

    sweep = None
    if args.full:
        sweep = []
        for i in (2, 3):
            name, n, k = SHAPES[i]
            for m in SWEEP_M:
                cfg, src = config(m, n, k)
                xm = [None] * len(SHAPES)
                xm[i] = torch.randn((m, k), generator=gen, device=dev).to(torch.float16)
                g, _ = capture([launcher(r % copies, i, xm, [cfg] * len(SHAPES)) for r in range(copies)])
                ms = median_replay_ms(g, copies)
                tflops = 2 * m * n * k / (ms * 1e-3) / 1e12
                gbps = bytes_moved(m, n, k) / (ms * 1e-3) / 1e9
                sweep.append({"layer": name, "m": m, "n": n, "k": k, "us": ms * 1e3, "tflops": tflops,
                              "frac_mfma": tflops / FP16_MFMA_PEAK_TFLOPS, "gbps": gbps,
                              "frac_hbm": gbps / HBM_PEAK_GBPS, "config": cfg.to_dict(), "config_source": src})
                log(f"  {name:13s} M={m:<5d} {ms * 1e3:9.2f} us {tflops:7.1f} TFLOP/s {gbps:7.0f} GB/s  {cfg}")
                del g, xm

    eager = eager_bench(layers, copies, xs, cfg1)
    vendor = vendor_bench(dev, gen)

    stack = None
    if not args.no_stack:
        stack = stack_bench(dev, gpu, STACK_M, args.tune)

    gate_n, gate_k = SHAPES[2][1], SHAPES[2][2]
    repack = {"gvalues_per_s": gate_n * gate_k / (rep_ms * 1e-3) / 1e9,
              "gbps": gate_n * gate_k / (rep_ms * 1e-3) / 1e9, "us": rep_ms * 1e3}
    cpu = None
    if not args.no_cpu:
        from tokenforge.kernels.hip.layout import tile_unpack

        t0 = time.perf_counter()
        layers_tf = [tuple(t.cpu() for t in tile_unpack(*layers[0][i], GROUP)) for i in range(len(SHAPES))]
        legs = cpu_baselines(layers_tf, gate_awq_host, norm_gamma.cpu())
        cpu = legs["decode"]
        for g in gemm:
            if g["m"] in (16, 256):
                g["cpu"] = legs[f"gemm_m{g['m']}"][g["layer"]]
        for r in norm:
            if r["t"] == legs["rmsnorm_t4096"]["t"]:
                r["cpu"] = legs["rmsnorm_t4096"]
        repack["cpu"] = legs["repack_gate_up"]
        log(f"cpu baselines ({cpu['cores']} threads, {cpu['cpu_model']}, {time.perf_counter() - t0:.1f}s): decode "
            f"{cpu['value']:.2f} GB/s; M=256 gate_up {legs['gemm_m256']['gate_up_proj']['tflops']:.2f} TFLOP/s, "
            f"down {legs['gemm_m256']['down_proj']['tflops']:.2f}; rmsnorm T=4096 "
            f"{legs['rmsnorm_t4096']['gbps']:.1f} GB/s; repack {legs['repack_gate_up']['gbps']:.2f} GB/s")
        del layers_tf

    result = {
        "metric": "W4A16 GEMV HBM GB/s at M=1 (% of peak) + GEMM TFLOP/s at M=256, Qwen-7B shapes",
        "value": value,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": elapsed_ms / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": "qwen2.5-7b decoder linears (qkv, o_proj, gate_up, down) W4A16 GEMV at M=1, "
                        "AWQ int4 g128, cold HBM",
            "m": 1,
            "group_size": GROUP,
            "layer_copies": copies,
            "bytes_per_step": step_bytes,
            "frac_of_hbm_peak": value / HBM_PEAK_GBPS,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"gate_up GEMV M=1 ({cfg1[2].kernel})",
            "achieved": dom["gbps"],
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": dom["gbps"] / HBM_PEAK_GBPS,
            "traffic": committed_traffic(cfg1[2].to_dict()),
            "bytes_per_launch": bytes_moved(1, gate_n, gate_k),
            "avg_launch_us": dom["us"],
            "config": cfg1[2].to_dict(),
            "config_source": src1[2],
        },
        "gemm_small_m": [g for g in gemm if g["m"] in SMALL_M],
        "gemm_m256": [g for g in gemm if g["m"] == 256],
        "gemm_m1024_m4096": [g for g in gemm if g["m"] > 256],
        "gemm_w4a8_fp8": gemm8,
        "rmsnorm_fp8": norm,
        "repack_gate_up": repack,
        "device_copy_gbps": copy_gbps,
        "per_shape": per_shape,
        "gemv_m2_m4": gemv_m24,
        "gemv_m8_m32": gemv_m8_m32,
        "vendor_fp16": vendor,
        "eager_op": eager,
        "stack": stack,
        "cpu_baseline": cpu,
        "cpu_decode_m8": legs["decode_m8"] if cpu is not None else None,
        "gpu": gpu,
        "env": fingerprint(),
    }
    result["regression"] = regression_check(result)
    if args.update_baseline is not None:
        update_baseline(result, args.reason, Path(args.update_baseline))
    if args.detail:
        detail = dict(result, gemm_sweep=sweep) if sweep is not None else result
        Path(args.detail).parent.mkdir(parents=True, exist_ok=True)
        Path(args.detail).write_text(json.dumps(detail, indent=1) + "\n")
    print(json.dumps(result), flush=True)
    reg = result["regression"]
    if args.check and reg is not None and reg.get("regressions"):
        for r in reg["regressions"]:
            log(f"REGRESSION {r['entry']}: {r['us']:.2f} us vs baseline {r['baseline_us']:.2f} us (+{r['slower_pct']:.1f}%)")
        return 1
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
