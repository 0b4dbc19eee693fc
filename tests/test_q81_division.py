"""The Q8_1 epilogue of the prefill attention rounds x / d with one division
per 32-value block and a two-fma correction of x * (1/d) (Markstein's
theorem).  This CPU test compiles the same arithmetic in C and compares it
with the division on random and adversarial (x, am) pairs over block maxima
from 2^-140 to 2^100: next to rounding ties, next to integers and at the
block maximum.  The GPU tests then check the kernel's Q8_1 planes bit for bit
against the oracle, which divides."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not installed")
def test_corrected_quotient_rounds_like_division(tmp_path):
    exe = tmp_path / "q81_div_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe),
                    os.path.join(HERE, "csrc", "q81_div_check.c"), "-lm"], check=True)
    for seed in (1, 2):
        out = subprocess.run([str(exe), "4000000", str(seed)], check=True, capture_output=True,
                             text=True).stdout.split()
        stats = dict(zip(out[0::2], map(int, out[1::2])))
        assert stats["n"] > 3_900_000
        assert stats["quotient_mismatches"] == 0, stats
        assert stats["round_mismatches"] == 0, stats
