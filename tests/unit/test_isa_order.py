"""The staged GEMMs wait for an x stage with ``s_waitcnt vmcnt(N)``, N = the loads issued after
that stage's LDS-destination loads. That count is only right if no later load is scheduled
above them, so every barrier of the generated gfx950 code must be followed by the x loads
(``buffer_load ... lds``) before any ordinary buffer load. (When the compiler hoisted weight
loads above them, workgroups read stages that had not landed.) Compiles the two sources to
assembly with the build's flags; needs hipcc, no GPU."""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

from tokenforge_amd import build

CSRC = Path(build.__file__).resolve().parent / "csrc"


def _order_after_barriers(asm: str) -> tuple[int, int]:
    """(barriers followed by an LDS load first, barriers followed by an ordinary load first)."""
    lines = asm.splitlines()
    good = bad = 0
    for i, line in enumerate(lines):
        if "s_barrier" not in line:
            continue
        for nxt in lines[i + 1:i + 400]:
            if "buffer_load" in nxt:
                if " lds" in nxt:
                    good += 1
                else:
                    bad += 1
                break
            if re.match(r"^\.LBB", nxt) or re.match(r"^\s*s_(c?branch|endpgm)", nxt) or "s_barrier" in nxt:
                break
    return good, bad


@pytest.mark.parametrize("source", ["gemm2.hip", "gemm3.hip"])
def test_x_stage_loads_lead_every_barrier_region(source: str, tmp_path: Path) -> None:
    try:
        cc = build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    if shutil.which(cc) is None and not Path(cc).exists():
        pytest.skip("hipcc not available")
    out = tmp_path / (source + ".s")
    flags = [f for f in build.HIPCC_FLAGS if f != "-fPIC"]
    subprocess.run([cc, *flags, "--cuda-device-only", "-S", str(CSRC / source), "-o", str(out)],
                   check=True, capture_output=True)
    good, bad = _order_after_barriers(out.read_text())
    assert good > 0, "no LDS-destination loads found after a barrier"
    assert bad == 0, f"{bad} barrier regions issue an ordinary load before the x-stage loads"
