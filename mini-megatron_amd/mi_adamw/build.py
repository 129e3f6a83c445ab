"""Compile libmi_adamw.so for gfx950 from csrc/ with hipcc, in place.

Run as ``python -m mi_adamw.build`` (with ``mini-megatron_amd`` on sys.path)
or through ``__graft_entry__.build()``.  The library lands next to this file,
where ``mi_adamw._lib`` loads it from.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
SOURCES = [os.path.join(HERE, "csrc", "mi_adamw.hip")]
INCLUDE = os.path.join(REPO, "include")
OUTPUT = os.path.join(HERE, "libmi_adamw.so")

# -ffp-contract=off: the kernels spell out every fused multiply-add themselves,
#   in the places torch-ROCm's kernels fuse, so the compiler must not add more.
# -packed-fp32-ops off: packed fp32 VALU forms are kept out of the code object.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build mi_adamw")
    return path


def build(verbose: bool = False) -> str:
    """Compile every source into libmi_adamw.so; returns the library path."""
    tmp = OUTPUT + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", INCLUDE, *SOURCES, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
