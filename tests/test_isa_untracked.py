"""The decode split kernel loads q, the norm weights and the new row with
untracked (inline-asm) vector loads issued ahead of the tile DMA, and awaits
them with one `s_waitcnt vmcnt(D*RPW)` that names their registers.  The
compiler does not know those registers are pending until that wait: any
instruction that touches them in between would read or clobber data still in
flight.  This CPU test compiles decode.hip for gfx950 (the library's flags) and
checks the generated assembly, in program order, for such an instruction, and
that the first vector-memory wait after the loads leaves the tile DMAs in flight.
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
        pending, in_asm, loads, first_wait = set(), False, 0, None
        for k, l in enumerate(body):
            if l.startswith(";;#ASMSTART"):
                in_asm = True
                continue
            if l.startswith(";;#ASMEND"):
                in_asm = False
                continue
            if in_asm and l.startswith("global_load_dwordx4") and "lds" not in l:
                pending |= _vregs(l.split()[1])
                loads += 1
                continue
            if "vmcnt(" in l:
                if pending and first_wait is None:
                    first_wait = int(re.search(r"vmcnt\((\d+)\)", l).group(1))
                pending = set()
                continue
            if l.startswith((".", ";")) or not l:
                continue
            hit = _vregs(l) & pending
            assert not hit, "%s line %d touches pending registers %s: %s" % (name, k, sorted(hit), l)
        assert loads == (20 if fused else 4), (name, loads)
        # D = 3 tiles of RPW = 4 rows per wave stay in flight
        assert first_wait == 12, (name, first_wait)
