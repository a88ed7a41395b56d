"""Cooperative launch planning (leo_amd/csrc/launch_plan.h): the runtime caps
the story lanes resident at once at the lanes one cooperative launch can hold,
and every planned grid for that many lanes fits the resident workgroup
capacity -- checked exhaustively over small device shapes by a host build of
the same header."""
from __future__ import annotations

import pathlib
import subprocess

ROOT = pathlib.Path(__file__).resolve().parents[1]


def test_launch_plans_fit_the_cooperative_capacity(tmp_path):
    exe = tmp_path / "launch_plan_check"
    subprocess.run(["g++", "-O2", "-std=c++17", f"-I{ROOT / 'leo_amd' / 'csrc'}",
                    str(ROOT / "tests" / "launch_plan_check.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=False, capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "checked" in out.stdout
