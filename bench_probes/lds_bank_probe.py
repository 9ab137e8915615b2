"""LDS bank-conflict probe of gfx950 (measurement only): the patterns, the build of the probe
program and the summary that becomes ``tests/golden/lds_bank_conflicts.json``.

The probe (``bench_probes/lds_bank_probe.hip``) runs one wave per pattern: each lane reads (or
writes) 16 bytes of LDS at the address the pattern gives it, 16 times. Under ``rocprofv3 --pmc
SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT`` each dispatch then yields the conflict cycles of one
16-byte access of that pattern (``SQ_LDS_BANK_CONFLICT / 16``; the probe's other LDS
instructions are linear and free of conflicts).

The patterns: the fragment reads and weight writes of the GEMM kernels under their old and
current LDS slot maps, linear reads and writes, one lane displaced onto lane 0's bank line for
each other lane (writes), and 200 random read and 200 random write patterns over 2 KB. The
bank model the GEMM slot maps rest on (``tests/unit/test_lds_bank_model.py``) is checked
against every measured pattern.

Usage::

    python bench_probes/lds_bank_probe.py build                      # bench_probes/lib/lds_bank_probe
    python bench_probes/lds_bank_probe.py patterns gpurun_out/lds_patterns.bin
    cd /tmp && export TMPDIR=/tmp && rocprofv3 --pmc SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT \\
        --output-format csv -d $R/gpurun_out/lds_probe -- $R/bench_probes/lib/lds_bank_probe \\
        $R/gpurun_out/lds_patterns.bin
    python bench_probes/lds_bank_probe.py summary gpurun_out/lds_probe
"""

from __future__ import annotations

import collections
import csv
import glob
import json
import random
import struct
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
FIXTURE = ROOT / "tests" / "golden" / "lds_bank_conflicts.json"
REPS = 16


def _row128(r: int, c: int) -> int:
    return r * 128 + (c & 7) * 16


def _row256(r: int, c: int) -> int:
    return r * 256 + (c & 15) * 16


def patterns() -> list[tuple[str, int, list[int]]]:
    """(name, mode: 0 read / 1 write, 64 byte addresses), in dispatch order."""
    pats: list[tuple[str, int, list[int]]] = []

    def add(name: str, mode: int, addrs: list[int]) -> None:
        assert len(addrs) == 64 and all(0 <= a < 16384 and a % 16 == 0 for a in addrs)
        pats.append((name, mode, addrs))

    s2_old = lambda r: (r >> 1) & 7  # noqa: E731
    s2_new = lambda r: ((r >> 1) & 7) ^ (((r >> 3) & 1) << 1)  # noqa: E731  (a candidate)
    for nm, s in (("old", s2_old), ("new", s2_new)):
        add(f"gemm2_read_{nm}", 0, [_row128(l & 31, (l >> 5) ^ s(l & 31)) for l in range(64)])
        wr = [_row128((l & 15) | ((l >> 5) << 4), (4 * ((l >> 4) & 1)) ^ s((l & 15) | ((l >> 5) << 4))) for l in range(64)]
        add(f"gemm2_write_{nm}", 1, wr)
        add(f"gemm2_writepat_as_read_{nm}", 0, wr)
    for nm, s in (("old", lambda r: r & 15), ("new", lambda r: r & 11)):
        add(f"gemm34_read_{nm}", 0, [_row256(l & 15, (4 * (l >> 4)) ^ s(l & 15)) for l in range(64)])
    for nm, s in (("old", lambda r: (r >> 1) & 7), ("new", lambda r: ((r & 3) << 1) ^ ((r >> 2) & 1))):
        rd = [_row128(l & 15, (2 * (l >> 4)) ^ s(l & 15)) for l in range(64)]
        add(f"gemm8_read_{nm}", 0, rd)
        add(f"gemm8_write_{nm}", 1, rd)
    add("linear_read", 0, [l * 16 for l in range(64)])
    add("linear_write", 1, [l * 16 for l in range(64)])
    for b in range(1, 64):
        add(f"phase_write_0_{b}", 1, [(1024 if l == b else l * 16) for l in range(64)])
    rng = random.Random(7)
    for i in range(200):
        add(f"rand_read_{i}", 0, [rng.randrange(128) * 16 for _ in range(64)])
    for i in range(200):
        add(f"rand_write_{i}", 1, [rng.randrange(128) * 16 for _ in range(64)])
    return pats


def write_patterns(path: str) -> None:
    pats = patterns()
    with open(path, "wb") as f:
        for _, mode, addrs in pats:
            f.write(struct.pack("<65I", mode, *addrs))
    print(f"wrote {path}: {len(pats)} patterns")


def build() -> None:
    sys.path.insert(0, str(ROOT))
    from tokenforge_amd import build as tb

    out = ROOT / "bench_probes" / "lib" / "lds_bank_probe"
    out.parent.mkdir(parents=True, exist_ok=True)
    flags = [f for f in tb.HIPCC_FLAGS if f not in ("-fPIC",)]
    subprocess.run([tb.hipcc(), *flags, "-o", str(out), str(ROOT / "bench_probes" / "lds_bank_probe.hip")], check=True)
    print(f"built {out}")


def summary(pmc_dir: str) -> None:
    """rocprofv3 counter CSV (one dispatch per pattern, in order) -> the golden fixture."""
    files = glob.glob(f"{pmc_dir}/**/*_counter_collection.csv", recursive=True)
    if len(files) != 1:
        raise SystemExit(f"expected one counter_collection.csv under {pmc_dir}, found {len(files)}")
    per: dict[int, dict[str, float]] = collections.defaultdict(dict)
    for row in csv.DictReader(open(files[0])):
        if "lds_pattern" in row["Kernel_Name"]:
            per[int(row["Dispatch_Id"])][row["Counter_Name"]] = float(row["Counter_Value"])
    pats = patterns()
    ids = sorted(per)
    if len(ids) != len(pats):
        raise SystemExit(f"{len(ids)} probe dispatches for {len(pats)} patterns")
    rows = []
    for (name, mode, addrs), did in zip(pats, ids):
        rows.append({"name": name, "mode": "read" if mode == 0 else "write", "slots": [a // 16 for a in addrs],
                     "conflict_cycles": per[did]["SQ_LDS_BANK_CONFLICT"] / REPS})
    doc = {"what": "SQ_LDS_BANK_CONFLICT cycles per 16-byte LDS access of one wave on MI355X (gfx950); "
                   "slots are 16-byte LDS slot indices of lanes 0..63",
           "made_by": "bench_probes/lds_bank_probe.py (module docstring)", "patterns": rows}
    FIXTURE.parent.mkdir(parents=True, exist_ok=True)
    FIXTURE.write_text(json.dumps(doc, separators=(",", ":")) + "\n")
    print(f"wrote {FIXTURE}: {len(rows)} patterns")


if __name__ == "__main__":
    cmd = sys.argv[1] if len(sys.argv) > 1 else ""
    if cmd == "build":
        build()
    elif cmd == "patterns" and len(sys.argv) == 3:
        write_patterns(sys.argv[2])
    elif cmd == "summary" and len(sys.argv) == 3:
        summary(sys.argv[2])
    else:
        sys.exit(__doc__)
