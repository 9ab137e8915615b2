"""Work-removal copies of the pipelined fp16 GEMM (``csrc/gemm2.hip``): measurement only, never
shipped, never loaded by the product.

Each copy takes one piece of work out of the kernel, so that the time of the rest can be set
beside the full kernel's; the outputs of a copy are wrong by design. The removals:

* ``dequant``: the packed weight words go to LDS as they are (no VALU dequantization);
* ``bstage``: no weight tile is dequantized or written to LDS (the buffers keep old data);
* ``xstage``: no x block is loaded into LDS after the prologue (the stages keep old data).

No removal changes an address: every access stays where the full kernel puts it, and the
barrier waits only wait for fewer loads, so every copy runs to completion.

Usage (the library build needs hipcc; the timing needs the GPU)::

    python bench_probes/work_removal.py build             # bench_probes/lib/libtokenforge_hip_<removal>.so
    python bench_probes/work_removal.py time > gpurun_out/work_removal.log
    python bench_probes/work_removal.py summary gpurun_out/work_removal.log   # profiles/gemm_m256_work_removal.md

``time`` runs one child process per library (the kernel library is chosen by
``TOKENFORGE_HIP_LIB`` when the package loads it) and times the shipped M=256 configs of
gate_up and down: the median over 5 replays of a HIP graph of 10 launches over 10 cold
weight copies, per launch, split-K reduce included.
"""

from __future__ import annotations

import json
import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
LIB_DIR = ROOT / "bench_probes" / "lib"
SHAPES = (("gate_up_proj", 37888, 3584), ("down_proj", 3584, 18944))
M = 256
GROUP = 128
COPIES = 10

# (text in gemm2.hip, replacement): each must occur exactly once.
REMOVALS: dict[str, tuple[str, str]] = {
    "dequant": (
        "        dequant_word(braw[slot][i][j], qp[i], uc, d);\n",
        "        d[0] = as_h2(braw[slot][i][j]); d[1] = as_h2(braw[slot][i][j] >> 1);\n"
        "        d[2] = as_h2(braw[slot][i][j] >> 2); d[3] = as_h2(braw[slot][i][j] >> 3);\n",
    ),
    "bstage": (
        "      if (kEvenB || tid + i * C::kThreads < C::kBChunks) {\n        h2 d[4];",
        "      if (false) {\n        h2 d[4];",
    ),
    "xstage": ("    issue_a(kb + S - 1, (st + S - 1) % S);\n", ""),
}


def lib_path(name: str) -> Path:
    return ROOT / "tokenforge_amd" / "lib" / "libtokenforge_hip.so" if name == "full" else LIB_DIR / f"libtokenforge_hip_{name}.so"


def build() -> None:
    sys.path.insert(0, str(ROOT))
    from tokenforge_amd import build as tb

    src = ROOT / "tokenforge_amd" / "csrc"
    for name, (old, new) in REMOVALS.items():
        # Two levels under the repository root, as csrc is: the sources include
        # ../../include/tokenforge_hip.h.
        tmp = ROOT / "bench_probes" / f"_src_{name}"
        if tmp.exists():
            shutil.rmtree(tmp)
        shutil.copytree(src, tmp)
        try:
            path = tmp / "gemm2.hip"
            text = path.read_text()
            if text.count(old) != 1:
                raise SystemExit(f"removal {name}: its text occurs {text.count(old)} times in gemm2.hip")
            path.write_text(text.replace(old, new))
            out = tb.build_library(sorted(tmp.glob("*.hip")), lib_path(name), tag=f"removal_{name}_")
            print(f"built {out}", flush=True)
        finally:
            shutil.rmtree(tmp)


def child() -> None:
    """Times the shipped M=256 configs with the library TOKENFORGE_HIP_LIB names; one JSON line."""
    sys.path.insert(0, str(ROOT))
    import functools
    import tempfile

    import torch

    os.environ["TOKENFORGE_CACHE_DIR"] = tempfile.mkdtemp()  # empty cache: the shipped table
    from tokenforge.kernels import autotune
    from tokenforge.kernels.device import gpu_identity
    from tokenforge.kernels.hip.w4a16 import w4a16_gemm

    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(5)
    rows = []
    for name, n, k in SHAPES:
        cfg = autotune.lookup(gpu_identity(dev), M, n, k, GROUP)
        layers = [autotune.synthetic_layer(n, k, GROUP, dev, seed=100 + i) for i in range(COPIES)]
        x = torch.randn((M, k), generator=gen, device=dev).to(torch.float16)
        fns = [functools.partial(w4a16_gemm, x, *lay, GROUP, cfg) for lay in layers]
        times = sorted(autotune.graph_bench(fns, reps=1) for _ in range(5))
        rows.append({"layer": name, "n": n, "k": k, "config": cfg.to_dict(), "us": times[2] * 1e3})
        del layers
        torch.cuda.empty_cache()
    print(json.dumps({"lib": os.environ.get("TOKENFORGE_HIP_LIB", ""), "rows": rows}), flush=True)


def time_all() -> int:
    for name in ("full", *REMOVALS):
        path = lib_path(name)
        if not path.exists():
            print(f"{path} missing: run `python bench_probes/work_removal.py build` first", file=sys.stderr)
            return 1
        env = dict(os.environ, TOKENFORGE_HIP_LIB=str(path))
        print(f"removal {name}", file=sys.stderr, flush=True)
        done = subprocess.run([sys.executable, __file__, "_child"], env=env, capture_output=True, text=True)
        if done.returncode != 0:
            sys.stderr.write(done.stderr[-2000:])
            return done.returncode
        line = [ln for ln in done.stdout.splitlines() if ln.startswith("{")][-1]
        rec = json.loads(line)
        rec["removal"] = name
        print(json.dumps(rec), flush=True)
    return 0


def summary(log: str) -> None:
    recs = [json.loads(ln) for ln in Path(log).read_text().splitlines() if ln.startswith("{")]
    by = {r["removal"]: {row["layer"]: row for row in r["rows"]} for r in recs}
    full = by["full"]
    out = [
        "# Where the M=256 fp16 GEMM's time goes: work-removal copies of the kernel",
        "",
        "Commands (on the MI355X box, fresh autotune cache: the configs are the shipped table's):",
        "",
        "```",
        "R=<repo root>",
        "python $R/bench_probes/work_removal.py build      # on the build host, before the GPU run",
        "python $R/bench_probes/work_removal.py time > $R/gpurun_out/work_removal.log",
        "python $R/bench_probes/work_removal.py summary $R/gpurun_out/work_removal.log",
        "```",
        "",
        "Each copy of the kernel library takes one piece of work out of `csrc/gemm2.hip` (module",
        "docstring of `bench_probes/work_removal.py`); its outputs are wrong by design. Times: median",
        "over 5 replays of a HIP graph of 10 launches over 10 cold weight copies, per launch (the",
        "split-K reduce of down included); synthetic layers, x ~ N(0, 1).",
        "",
        "| removal | " + " | ".join(f"{layer} us | saved" for layer, _, _ in SHAPES) + " |",
        "|---|" + "---:|---:|" * len(SHAPES),
    ]
    for name in ("full", *REMOVALS):
        cells = []
        for layer, _, _ in SHAPES:
            us = by[name][layer]["us"]
            saved = full[layer]["us"] - us
            pct = saved / full[layer]["us"] * 100
            cells.append(f"{us:.2f} | " + ("-" if name == "full" else f"{saved:.2f} ({pct:.0f}%)"))
        out.append(f"| {name} | " + " | ".join(cells) + " |")
    cfgs = {layer: full[layer]["config"] for layer, _, _ in SHAPES}
    out += ["", "Configs: " + "; ".join(f"{layer} `{json.dumps(c)}`" for layer, c in cfgs.items())]
    path = ROOT / "profiles" / "gemm_m256_work_removal.md"
    path.write_text("\n".join(out) + "\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    cmd = sys.argv[1] if len(sys.argv) > 1 else ""
    if cmd == "build":
        build()
    elif cmd == "time":
        sys.exit(time_all())
    elif cmd == "_child":
        child()
    elif cmd == "summary" and len(sys.argv) == 3:
        summary(sys.argv[2])
    else:
        sys.exit(__doc__)
