"""The decode split kernel loads q, the norm weights and the new row with
untracked (inline-asm) vector loads issued ahead of the tile DMA, and awaits
them with one `s_waitcnt vmcnt(D*RPW)` that names their registers.  The
compiler does not know those registers are pending until that wait: any
instruction that touches them in between would read or clobber data still in
flight.  This CPU test compiles decode.hip for gfx950 (the library's flags) and
checks the generated assembly along every control-flow path (branches
followed, so the early return of a slice with no positions is covered as well
as the tile loop) for such an instruction, and that the first vector-memory
wait after the loads leaves the tile DMAs in flight.
"""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "lfm2-ampere_amd")
HIPCC = "/opt/rocm/bin/hipcc"
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-DLK_ATTN_SPLIT=256", "-DLK_ATTN_TARGET_N=16", "-DLK_ATTN_SPLIT_MIN=8",
         "-DLK_DEC_TILE=16", "-DLK_DEC_NBUF=4", "-DLK_DEC_ABLATE=0"]


def _vregs(text):
    out = set()
    for m in re.finditer(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b", text):
        if m.group(3):
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def _check_paths(name, body):
    """Dataflow over the kernel's instructions: the set of registers of
    untracked loads still in flight at each instruction, joined over every
    path that reaches it; any instruction other than a vector-memory wait that
    names one of them is a hazard.  Returns (number of untracked loads, vmcnt
    of the first wait that retires them)."""
    ins, labels = [], {}
    in_asm = False
    for l in body:
        if l.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if l.startswith(";;#ASMEND"):
            in_asm = False
            continue
        m = re.match(r"^(\.?[A-Za-z_][\w.$]*):", l)
        if m:
            labels[m.group(1)] = len(ins)
            continue
        if l.startswith(";") or not l or (l.startswith(".") and not in_asm):
            continue
        ins.append((l.split(";")[0].strip(), in_asm))
    loads = sum(1 for t, a in ins if a and t.startswith("global_load_dwordx4") and "lds" not in t)
    state = [None] * (len(ins) + 1)
    state[0] = frozenset()
    work, first_wait = [0], None
    while work:
        k = work.pop()
        if k >= len(ins):
            continue
        t, a = ins[k]
        pend = state[k]
        op = t.split()[0]
        if a and op == "global_load_dwordx4" and "lds" not in t:
            out = pend | _vregs(t.split(None, 1)[1].split(",")[0])
        elif "vmcnt(" in t:
            if pend and first_wait is None:
                first_wait = int(re.search(r"vmcnt\((\d+)\)", t).group(1))
            out = frozenset()
        else:
            hit = _vregs(t) & pend
            assert not hit, "%s: %s touches registers of loads in flight %s" % (name, t, sorted(hit))
            out = pend
        succ = []
        if op == "s_endpgm":
            succ = []
        elif op == "s_branch":
            succ = [labels[t.split()[1]]]
        elif op.startswith("s_cbranch"):
            succ = [k + 1, labels[t.split()[1]]]
        else:
            succ = [k + 1]
        for j in succ:
            new = out if state[j] is None else (state[j] | out)
            if state[j] is None or new != state[j]:
                state[j] = new
                work.append(j)
    return loads, first_wait


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_untracked_loads_untouched_until_their_wait(tmp_path):
    asm = tmp_path / "decode.s"
    subprocess.run([HIPCC, *FLAGS, "--offload-device-only", "-S", "-x", "hip",
                    os.path.join(PKG, "csrc", "decode.hip"), "-o", str(asm)],
                   check=True, cwd=PKG, capture_output=True)
    txt = asm.read_text()
    for fused in (0, 1):
        name = "_Z15lk_k_attn_splitILb%dE" % fused
        i = txt.index("\n" + name) + 1
        body = [l.strip() for l in txt[i:txt.index(".Lfunc_end", i)].split("\n")]
        loads, first_wait = _check_paths(name, body)
        assert loads == (20 if fused else 4), (name, loads)
        # D = 3 tiles of RPW = 4 rows per wave stay in flight
        assert first_wait == 12, (name, first_wait)
