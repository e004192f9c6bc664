"""The division-free int8 code of the activation quantisers
(webyiq_amd/csrc/quant_code.hpp) equals rint(v / d) with an IEEE quotient:
the same header compiled for the host with g++ and checked over random and
half-integer-boundary inputs (tests/quant_code_check.cpp)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "webyiq_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_quant_code_matches_ieee_division(tmp_path):
    exe = str(tmp_path / "quant_code_check")
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-fno-fast-math", "-DWQ_HD=",
                    "-I", CSRC, os.path.join(HERE, "quant_code_check.cpp"), "-o", exe], check=True)
    out = subprocess.run([exe], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "mismatches 0" in out.stdout
