"""The staged GEMMs wait for an x stage with ``s_waitcnt vmcnt(N)``, N = the loads issued after
that stage's LDS-destination loads, counted by hand in the source. Two checks on the generated
gfx950 code: every barrier is followed by the x loads (``buffer_load ... lds``) before any
ordinary buffer load (when the compiler hoisted weight loads above them, workgroups read
stages that had not landed), and every barrier's N is at most the loads actually issued after
the stage it guards, on every control-flow path to it. Compiles the sources to assembly with
the build's flags; needs hipcc, no GPU."""

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


@pytest.mark.parametrize("source", ["gemm2.hip", "gemm3.hip", "gemm4.hip"])
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


# ------------------------------------------------------------------------ wait counts

_VMEM = re.compile(r"^(buffer|global|flat|scratch)_(load|store|atomic)")
_WAIT = re.compile(r"^s_waitcnt\b.*\bvmcnt\((\d+)\)")
_KERNEL = re.compile(r"^(_Z\w*(gemm2_kernel|gemm3_kernel|gemm4_kernel|gemm8_kernel|gemm2pc_kernel|gemm8pc_kernel)I(\w*?)EEv\w*):")
_JUMP = re.compile(r"^s_(c?branch)\w*\s+(\.LBB\w+)")
_INF = float("inf")


def _instructions(body: list[str]) -> list[str]:
    """Instructions and block labels of one function; comments and directives dropped."""
    out = []
    for raw in body:
        line = raw.split(";", 1)[0].strip()
        if line.startswith("."):
            if re.match(r"^\.LBB\w+:$", line):
                out.append(line)
            continue
        if line:
            out.append(line)
    return out


def _stages(kernel: str, template_args: str) -> int:
    """S: the fifth integer template argument of gemm2/3/8_kernel and of the producer / consumer
    forms, the fourth of gemm4_kernel."""
    return [int(v) for v in re.findall(r"Li(\d+)E", template_args + "E")][3 if kernel == "gemm4_kernel" else 4]


def _block_waits(ins: list[str]) -> dict[int, int]:
    """Index of each block barrier -> N of the ``s_waitcnt vmcnt(N)`` right before it."""
    out = {}
    for i, line in enumerate(ins):
        if line.startswith("s_barrier"):
            k = i - 1
            while k >= 0 and ins[k].endswith(":"):
                k -= 1
            m = _WAIT.match(ins[k]) if k >= 0 else None
            if m:
                out[i] = int(m.group(1))
    return out


_SREG = re.compile(r"\bs\[(\d+):(\d+)\]|\bs(\d+)\b")
_VCC_WRITERS = re.compile(r"^v_(cmp|cmpx|add_co|sub_co|subrev_co|addc|subb|subbrev|div_scale|div_fmas)")


def _sregs(text: str) -> set[int]:
    out: set[int] = set()
    for a, b, one in _SREG.findall(text):
        out |= set(range(int(a), int(b) + 1)) if a else {int(one)}
    return out


def _wait_checks(ins: list[str], stages: int, consumers: set[int] | None = None) -> list[tuple[int, int, float]]:
    """(barrier index, its vmcnt N, the fewest vector-memory instructions issued after the last
    x load of the stage that barrier guards, over every path that reaches it; -1 where a path
    has no stage left for it).

    Loads return in order, so the wait guarantees the stage iff N <= that count. The code is
    walked forward over every control-flow path, carrying the x stages issued and not yet
    guarded, oldest first, each with the number of vector-memory instructions issued since its
    last load (capped past the largest N). The x loads (``buffer_load ... lds``) before the first
    barrier are S - 1 stages of equal size issued in order; between two later barriers they are
    one stage (or none: a barrier in the middle of an iteration may guard a stage issued before
    the previous one). Each barrier guards the oldest stage still pending, so the n-th barrier on
    a path guards the n-th stage issued. A conditional branch is followed both ways unless its
    outcome is fixed on that path: ``s_cbranch_vccz``/``vccnz`` after
    ``s_andn2_b64 vcc, exec, s[a:b]`` with s[a:b] set by ``s_mov_b64`` to 0 or -1 (exec is
    nonzero: the stage loads are issued by the whole wave). The compiler writes such a pair of
    correlated branches around the two copies of a load it duplicates (an in-range and an
    out-of-range offset); following both ways would count a path that skips both copies.

    With ``consumers`` (a set, filled here), the producer / consumer forms: a path that reaches
    a barrier without having issued any x load is a consumer wave's (those waves load nothing
    and wait on the producers' barrier): it is followed on as a consumer path and every barrier
    it reaches is collected in ``consumers``. The walk does not know the wave-uniform role
    branch, so it also follows role-mixing paths no wave takes; those end up consumer paths as
    well. Every barrier a producer path reaches (one that issued the prologue's x stages) is
    checked as above; the caller drops only the barriers no producer path reaches."""
    labels = {l[:-1]: i for i, l in enumerate(ins) if l.endswith(":")}
    waits = _block_waits(ins)
    cap = max(waits.values(), default=0) + 1  # counts past every N compare alike
    # the pairs some s_andn2_b64 vcc, exec, s[a:b] reads: the only constants worth a state
    wanted = {m.group(1) for m in (re.match(r"^s_andn2_b64 vcc, exec, (s\[\d+:\d+\])$", l) for l in ins) if m}
    # live[pc]: a barrier can still be reached from pc (past the last one nothing is checked)
    live = [pc in waits for pc in range(len(ins))]
    changed = True
    while changed:
        changed = False
        for pc in range(len(ins) - 1, -1, -1):
            if live[pc]:
                continue
            op = ins[pc].split()[0]
            m = _JUMP.match(ins[pc])
            nxt = [] if op in ("s_endpgm", "s_setpc_b64", "s_branch") else [pc + 1]
            if m:
                nxt.append(labels[m.group(2)])
            if any(n < len(ins) and live[n] for n in nxt):
                live[pc] = changed = True
    best: dict[int, float] = {}
    seen: set[tuple] = set()
    # (pc, constant pairs, vcc: None unknown / 0 / 1, pending stage counters, this region's
    # x-load counters, in the prologue, a consumer path)
    todo: list[tuple] = [(0, (), None, (), (), True, False)]
    while todo:
        state = todo.pop()
        if state in seen:
            continue
        seen.add(state)
        pc, consts, vcc, pending, region, pro, cons = state
        cmap = dict(consts)
        while pc < len(ins) and live[pc]:
            line = ins[pc]
            if line.endswith(":"):
                key = (pc + 1, tuple(sorted(cmap.items())), vcc, pending, region, pro, cons)
                if key in seen:
                    break
                seen.add(key)
                pc += 1
                continue
            op = line.split()[0]
            args = [a.strip() for a in line[len(op):].split(",")]
            if pc in waits:
                if consumers is not None and (cons or (pro and not region)):
                    consumers.add(pc)  # a consumer wave's barrier: it issues no loads
                    # a consumer path carries no state: every such walk from a pc is the same
                    cons, pending, region, pro, cmap, vcc = True, (), (), False, {}, None
                    pc += 1
                    continue
                if pro:
                    if not region or len(region) % (stages - 1):
                        best[pc] = -1
                        break
                    per = len(region) // (stages - 1)
                    pending = tuple(region[(k + 1) * per - 1] for k in range(stages - 1))
                    pro = False
                elif region:
                    pending = pending + (region[-1],)
                region = ()
                if not pending:
                    best[pc] = -1  # no stage issued for this barrier
                    break
                best[pc] = min(best.get(pc, _INF), pending[0])
                pending = pending[1:]
                pc += 1
                continue
            if _VMEM.match(line) and not cons:
                pending = tuple(min(c + 1, cap) for c in pending)
                region = tuple(min(c + 1, cap) for c in region)
                if " lds" in line:
                    # the prologue's stages need each load's counter; an iteration's, its last
                    region = region + (0,) if pro else (0,)
            if cons:
                pass
            elif op == "s_mov_b64" and args[0] in wanted and args[1] in ("0", "-1"):
                cmap = {k: v for k, v in cmap.items() if not (_sregs(k) & _sregs(args[0]))}
                cmap[args[0]] = int(args[1])
            elif op == "s_andn2_b64" and args[:2] == ["vcc", "exec"] and args[2] in cmap:
                vcc = 0 if cmap.pop(args[2]) == -1 else 1
            else:
                touched = _sregs(line)
                if touched:
                    cmap = {k: v for k, v in cmap.items() if not (_sregs(k) & touched)}
                if ("vcc" in line or _VCC_WRITERS.match(op)) and not op.startswith("s_cbranch_vcc"):
                    vcc = None
            if op in ("s_endpgm", "s_setpc_b64"):
                break
            m = _JUMP.match(line)
            if m:
                target = labels[m.group(2)]
                if op == "s_branch":
                    pc = target
                    continue
                taken = {"s_cbranch_vccnz": vcc, "s_cbranch_vccz": None if vcc is None else 1 - vcc}.get(op)
                if taken != 0:
                    todo.append((target, tuple(sorted(cmap.items())), vcc, pending, region, pro, cons))
                if taken == 1:
                    break
            pc += 1
    return [(b, n, best.get(b, _INF)) for b, n in sorted(waits.items())]


def _kernel_checks(asm: str) -> dict[str, list[tuple[int, int, float]]]:
    lines = asm.splitlines()
    out = {}
    i = 0
    while i < len(lines):
        m = _KERNEL.match(lines[i])
        if not m:
            i += 1
            continue
        j = i + 1
        while j < len(lines) and not lines[j].startswith(".Lfunc_end"):
            j += 1
        ins = _instructions(lines[i + 1:j])
        if "pc_kernel" in m.group(2):
            consumers: set[int] = set()
            rows = _wait_checks(ins, _stages(m.group(2), m.group(3)), consumers)
            # the barriers only consumer paths reach; every other one is checked
            out[m.group(1)] = [row for row in rows if not (row[0] in consumers and row[2] == _INF)]
            assert consumers and len(out[m.group(1)]) < len(rows), f"{m.group(1)}: no consumer barrier found"
        else:
            out[m.group(1)] = _wait_checks(ins, _stages(m.group(2), m.group(3)))
        i = j
    return out


@pytest.mark.parametrize("source", ["gemm2.hip", "gemm3.hip", "gemm4.hip", "gemm8.hip"])
def test_stage_waits_cover_the_stage_loads(source: str, tmp_path: Path) -> None:
    """Every block barrier's vmcnt(N) is at most the loads issued after the x stage its
    iteration reads, on every path to it (loop, prologue and the odd tail iteration), so the
    stage has landed when the barrier is passed."""
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
    checks = _kernel_checks(out.read_text())
    assert checks, "no staged GEMM kernels found"
    for name, rows in checks.items():
        assert len(rows) >= 2, f"{name}: expected a loop barrier and the tail barrier"
        for b, n, after in rows:
            assert after != -1, f"{name}: a path to the barrier at {b} issues no x stage"
            assert after != _INF, f"{name}: no path reaches the barrier at {b}"
            assert n <= after, f"{name}: barrier at {b} waits vmcnt({n}), only {after} loads follow the stage"


_X = "buffer_load_dwordx4 v1, s[8:11], 0 offen lds"
_W = "buffer_load_dword v2, v3, s[16:19], 0 offen"


def _toy(loop_wait: int, tail_wait: int, guard_loop_load: bool = False) -> list[str]:
    """Two stages (S = 2), one x load per stage: prologue x + 2 weight loads, a loop whose
    iteration is barrier, x, weight (optionally behind an execz branch), and a tail iteration."""
    body = [_X, _W, _W, ".LBB0_1:", f"s_waitcnt vmcnt({loop_wait}) lgkmcnt(0)", "s_barrier", _X]
    if guard_loop_load:
        body += ["s_cbranch_execz .LBB0_2", _W, ".LBB0_2:"]
    else:
        body += [_W]
    body += ["s_cbranch_scc0 .LBB0_1", f"s_waitcnt vmcnt({tail_wait}) lgkmcnt(0)", "s_barrier", _X, "s_endpgm"]
    return body


def test_wait_check_on_a_toy_loop() -> None:
    """The analysis on hand-written code: the loop barrier from the prologue (2 loads after the
    stage) and from the back edge (1), the tail barrier after the loop (1); a wait one too
    permissive, and a load that may be skipped, are caught."""
    ok = _wait_checks(_instructions(_toy(1, 1)), 2)
    assert [(n, a) for _, n, a in ok] == [(1, 1), (1, 1)]
    loose = _wait_checks(_instructions(_toy(2, 1)), 2)
    assert loose[0][1] > loose[0][2]
    loose_tail = _wait_checks(_instructions(_toy(1, 2)), 2)
    assert loose_tail[1][1] > loose_tail[1][2]
    guarded = _wait_checks(_instructions(_toy(1, 1, guard_loop_load=True)), 2)
    assert [a for _, _, a in guarded] == [0, 0]
    s3 = [_X, _X, _W, ".LBB0_1:", "s_waitcnt vmcnt(2) lgkmcnt(0)", "s_barrier", _X, _W,
          "s_cbranch_scc0 .LBB0_1", "s_endpgm"]
    # S = 3: from the prologue the stage read is the first of its two x loads (x, weight after
    # it: 2); around the loop it was issued two iterations back (weight, x, weight: 3).
    assert [a for _, _, a in _wait_checks(_instructions(s3), 3)] == [2]
    s3[4] = "s_waitcnt vmcnt(3) lgkmcnt(0)"
    assert _wait_checks(_instructions(s3), 3)[0][1] > 2


def test_wait_check_follows_correlated_branches() -> None:
    """A load duplicated under two correlated branches (the compiler's form for an offset
    selected between a computed and an out-of-range value): exactly one copy issues on every
    path, so one load follows the loop's x stage; with the pair's value unknown, the path that
    skips both copies counts and the wait is reported too long."""
    def body(set_known: bool) -> list[str]:
        arm_taken = "s_mov_b64 s[18:19], -1" if set_known else "s_and_b64 s[18:19], s[2:3], s[4:5]"
        arm_fall = "s_mov_b64 s[18:19], 0" if set_known else "s_or_b64 s[18:19], s[2:3], s[4:5]"
        return [_X, _W, _W, ".LBB0_1:", "s_waitcnt vmcnt(1) lgkmcnt(0)", "s_barrier",
                "s_cmp_ge_i32 s41, s34", _X, arm_taken, "s_cbranch_scc0 .LBB0_2",
                arm_fall, _W, ".LBB0_2:", "s_andn2_b64 vcc, exec, s[18:19]", "v_add_u32_e32 v5, s6, v7",
                "s_cbranch_vccnz .LBB0_3", _W, ".LBB0_3:", "s_cbranch_scc0 .LBB0_1", "s_endpgm"]
    assert [(n, a) for _, n, a in _wait_checks(_instructions(body(True)), 2)] == [(1, 1)]
    assert [(n, a) for _, n, a in _wait_checks(_instructions(body(False)), 2)] == [(1, 0)]


def test_wait_check_with_a_barrier_inside_the_iteration() -> None:
    """The wave-tile GEMM's order: the prologue issues S - 1 = 2 stages and the weights, waits for
    the first stage at a barrier; each iteration then waits (mid-iteration) for the stage after
    it, which no x load separates from the previous barrier, issues the next stage and then the
    weights. The n-th barrier guards the n-th stage: from the prologue 2 loads follow the second
    stage (the weights), around the loop 1 (the weights after the stage issued one iteration
    back); a wait one too permissive is caught."""
    def body(loop_wait: int) -> list[str]:
        return [_X, _X, _W, _W, "s_waitcnt vmcnt(3) lgkmcnt(0)", "s_barrier", ".LBB0_1:",
                f"s_waitcnt vmcnt({loop_wait}) lgkmcnt(0)", "s_barrier", _X, _W, "s_cbranch_scc0 .LBB0_1",
                "s_endpgm"]
    rows = _wait_checks(_instructions(body(1)), 3)
    assert [(n, a) for _, n, a in rows] == [(3, 3), (1, 1)]
    loose = _wait_checks(_instructions(body(2)), 3)
    assert loose[1][1] > loose[1][2]
