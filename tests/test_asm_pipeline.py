"""The prefill GEMMs' load pipeline is inline asm: the compiler does not know that an asm
load's destination registers fill in later, so a copy or other use of them that it places
before the kernel's explicit `s_waitcnt vmcnt` reads stale values (no error, wrong output).
This compiles prefill.hip to gfx950 assembly (CPU only) and checks every grouped-GEMM kernel
along each fall-through path: after a vector load, no instruction touches its destination
registers until an `s_waitcnt vmcnt(N)` with at least N vector memory operations issued
since the load (vector memory completes in issue order, so that wait covers it).  Paths are
followed in program order through conditional branches (their fall-through is a real path)
and end at an unconditional branch."""
import os
import re
import shutil
import subprocess
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
from tarfa_amd import build as B  # noqa: E402

LOAD = re.compile(r"^(global|buffer)_load_(dword\w*|ushort|ubyte|short|sbyte)\s+(v\[\d+:\d+\]|v\d+)")
REG = re.compile(r"v\[(\d+):(\d+)\]|\b(v\d+)\b")


def _regs(text):
    out = set()
    for a, b, c in REG.findall(text):
        if c:
            out.add(int(c[1:]))
        else:
            out |= set(range(int(a), int(b) + 1))
    return out


def early_uses(lines):
    """(load, first instruction touching its destination before a covering wait) pairs."""
    code = [l.split(";")[0].strip() for l in lines]
    bad = []
    for i, l in enumerate(code):
        m = LOAD.match(l)
        if not m or "_lds" in l:
            continue
        dst = _regs(m.group(3))
        issued = 0                       # vector memory operations issued after the load
        for l2 in code[i + 1:]:
            if l2.startswith("s_waitcnt") and "vmcnt" in l2:
                if issued >= int(re.search(r"vmcnt\((\d+)\)", l2).group(1)):
                    break
                continue
            if l2.startswith(("s_endpgm", "s_branch", "s_setpc")):
                break
            if not l2 or l2.endswith(":") or l2.startswith((".", "s_")):
                continue
            op, _, ops = l2.partition(" ")
            if op.startswith(("global_", "buffer_", "flat_", "scratch_")):
                issued += 1
            if _regs(ops) & dst:
                bad.append((l, l2))
                break
    return bad


def test_checker_flags_a_copy_before_the_wait():
    load = "global_load_dwordx2 v[194:195], v154, s[76:77]"
    covered = [load, "global_load_dword v7, v1, s[0:1]", "s_waitcnt vmcnt(1)", "v_mov_b32_e32 v3, v194"]
    early = [load, "global_load_lds_dwordx4 v206, s[2:3]", "v_mov_b32_e32 v3, v194", "s_waitcnt vmcnt(0)"]
    short = [load, "global_load_dword v7, v1, s[0:1]", "s_waitcnt vmcnt(2)", "v_mov_b32_e32 v3, v195"]
    waw = ["global_load_dword v10, v1, s[0:1]", "v_mov_b32_e32 v10, 0", "s_waitcnt vmcnt(0)"]
    other = [load, "v_mov_b32_e32 v3, v196", "s_branch .LBB0_1", "v_mov_b32_e32 v3, v194"]
    assert early_uses(covered) == []
    assert early_uses(early) == [(load, early[2])]
    assert early_uses(short) == [(load, short[3])]     # the wait leaves this load outstanding
    assert early_uses(waw) == [(waw[0], waw[1])]
    assert early_uses(other) == []                     # past an unconditional branch: another path


@pytest.mark.skipif(not shutil.which(B.HIPCC) and not os.path.exists(B.HIPCC), reason="hipcc not installed")
def test_grouped_gemm_pipeline_loads_untouched_before_a_wait(tmp_path):
    out = tmp_path / "prefill.s"
    r = subprocess.run([B.HIPCC, *B.CFLAGS, "--cuda-device-only", "-S", os.path.join(B.CSRC, "prefill.hip"),
                        "-o", str(out)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    asm = out.read_text()
    names = re.findall(r"^(_ZN4tmoe\d+k_grouped_gemm\w*):", asm, re.M)
    assert any("gemm_pI" in n for n in names) and any("gemm_wI" in n for n in names), names
    problems = {}
    for n in names:
        i = asm.index(n + ":")
        body = asm[i:asm.index(".Lfunc_end", i)].splitlines()
        if early_uses(body):
            problems[n] = early_uses(body)[:3]
    assert not problems, problems
