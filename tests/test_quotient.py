"""The fp8 row quantiser divides by the row scale with a reciprocal and one
Markstein correction instead of an IEEE division (aps2026_amd/csrc/quant.hip,
quotient()).  tests/cpp/quotient_check.c restates that arithmetic in C and
compares the resulting e4m3 code with the code of the IEEE quotient for every
bf16 amax and (here) every 64th bf16 value: the codes must agree everywhere,
while the uncorrected product must not (so the check can fail).  Run the
program with stride 1 for the exhaustive 1.07e9-pair check."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "cpp", "quotient_check.c")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_markstein_quotient_gives_the_ieee_e4m3_code(tmp_path):
    exe = str(tmp_path / "quotient_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, SRC, "-lm"], check=True)
    res = subprocess.run([exe, "64"], capture_output=True, text=True, timeout=300)
    m = re.search(r"pairs (\d+) mismatches (\d+) plain-product mismatches (\d+)", res.stdout)
    assert m, res.stdout + res.stderr
    pairs, bad, bad_plain = map(int, m.groups())
    assert pairs > 10_000_000
    assert bad == 0 and res.returncode == 0, res.stdout
    assert bad_plain > 0  # the correction step matters: the check can fail
