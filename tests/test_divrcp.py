"""The division used by the GPTQ column loop and the ladder fit (hi2_amd/csrc/divrcp.h)
against IEEE division, on the host (CPU test).

The kernels divide through a precomputed reciprocal (Markstein's iteration), which is
exact only for operands whose intermediates stay normal; ``div_rcp`` adds a range test
with an IEEE fallback, ``div_rcp_code`` (quotients only rounded to a clamped code) a
branch-free guard.  The same header is compiled here with g++ (fma, no contraction) and
checked on random operands of every exponent and on the cases the iteration alone gets
wrong: subnormal and zero numerators, subnormal quotients, overflow, inf and NaN.
"""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_div_rcp_matches_ieee_division(tmp_path):
    exe = tmp_path / "divrcp_check"
    subprocess.run(["g++", "-O2", "-mfma", "-ffp-contract=off", "-std=c++17",
                    os.path.join(HERE, "native", "divrcp_check.cpp"), "-o", str(exe)],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
