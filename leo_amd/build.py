"""Build the native pieces of leo_amd.

    python -m leo_amd.build            # libleo_hip.so (gfx950) + the CPU oracle

libleo_hip.so holds the HIP kernels, the host runtime and the C-ABI of
include/leo_hip.h. It is built in-tree (leo_amd/_lib/) so that it travels with
the repository to the GPU box. Every HIP translation unit is compiled with
-ffp-contract=off (the kernels must round exactly where Leo's CPU executor
rounds) and with packed-FP32 instructions disabled.
"""
from __future__ import annotations

import os
import pathlib
import shutil
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parents[1]
CSRC = ROOT / "leo_amd" / "csrc"
LIB_DIR = ROOT / "leo_amd" / "_lib"
LIB = LIB_DIR / "libleo_hip.so"
BUILD = ROOT / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-pthread", "-ffp-contract=off", "-Wall", "-Wextra",
             f"-I{ROOT / 'include'}", f"-I{CSRC}"]


def _run(cmd):
    print("+ " + " ".join(str(c) for c in cmd), flush=True)
    subprocess.run([str(c) for c in cmd], check=True)


def build_library() -> pathlib.Path:
    BUILD.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    objects = []
    for src in ("leo_kernels.hip", "leo_runtime.hip"):
        obj = BUILD / (src + ".o")
        _run([HIPCC, *HIP_FLAGS, "-c", CSRC / src, "-o", obj])
        objects.append(obj)
    for src in ("host_model.cpp", "formats.cpp"):
        obj = BUILD / (pathlib.Path(src).stem + ".o")
        _run([os.environ.get("CXX", "g++"), *CXX_FLAGS, "-c", CSRC / src, "-o", obj])
        objects.append(obj)
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", *objects, "-o", tmp])
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> pathlib.Path:
    _run(["make", "-s", "-B", "-C", ROOT / "oracle"])
    return ROOT / "oracle" / "liboracle.so"


def main() -> int:
    subprocess.run([sys.executable, str(CSRC / "gen_abi.py"), "--check"], check=True)
    build_library()
    if shutil.which("make"):
        build_oracle()
    return 0


if __name__ == "__main__":
    sys.exit(main())
