"""The kernels' division by launch-constant divisors (leo_amd/csrc/fast_div.h:
multiply by a rounded-up reciprocal, then shift) equals integer division for
every dividend below 2^31 -- checked by brute force over small divisors, powers
of two and their neighbours, and random divisors at edge and random dividends.
The header is compiled for the host with g++ (the device build compiles the
same source)."""
from __future__ import annotations

import pathlib
import subprocess

ROOT = pathlib.Path(__file__).resolve().parents[1]


def test_fast_div_matches_integer_division(tmp_path):
    exe = tmp_path / "fastdiv_check"
    subprocess.run(["g++", "-O2", "-std=c++17", f"-I{ROOT / 'leo_amd' / 'csrc'}",
                    str(ROOT / "tests" / "fastdiv_check.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=False, capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "checked" in out.stdout
