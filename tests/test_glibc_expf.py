"""The device's exp (leo_amd/csrc/glibc_expf.h) is bit-identical to the host
glibc expf that Leo's CPU softmax calls (runtime.rs:1169-1188, Rust f32::exp),
over every float of the softmax's domain [-103.97, 0]. The header is compiled
for the host with g++ (the device build compiles the same source)."""
from __future__ import annotations

import pathlib
import subprocess

ROOT = pathlib.Path(__file__).resolve().parents[1]


def test_restated_expf_matches_glibc_everywhere(tmp_path):
    exe = tmp_path / "expf_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-mfma",
                    f"-I{ROOT / 'leo_amd' / 'csrc'}", str(ROOT / "tests" / "expf_check.cpp"), "-o", str(exe), "-lm"],
                   check=True)
    out = subprocess.run([str(exe)], check=False, capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "checked" in out.stdout
