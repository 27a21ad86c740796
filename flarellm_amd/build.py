"""Build the HIP backend library (libflare_hip.so) in-tree for gfx950.

Run as ``python -m flarellm_amd.build`` or through ``__graft_entry__.build()``.
Compiles every time it is called (hipcc cross-compiles without a GPU).
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libflare_hip.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -ffp-contract=off: the reference (Rust) never fuses a*b+c; per-block float
# terms must be formed with the same roundings.  The packed-fp32 feature is
# disabled for all device code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unknown-pragmas", "-Wno-unused-result",
]
CXX_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-fopenmp", "-ffp-contract=off"]


def _run(cmd: list[str]) -> None:
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    hip_obj = os.path.join(BUILD, "flare_hip.o")
    syn_obj = os.path.join(BUILD, "synth.o")
    _run([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, "flare_hip.hip"), "-o", hip_obj])
    _run(["g++", *CXX_FLAGS, "-c", os.path.join(CSRC, "synth.cpp"), "-o", syn_obj])
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", hip_obj, syn_obj, "-lgomp", "-o", tmp])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
