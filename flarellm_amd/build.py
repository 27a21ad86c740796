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


# Per-source flags.  verify.hip: MFMA results in VGPRs (no accumulator-
# register copies before the fp32 block terms of the GEMM epilogues).
SOURCE_FLAGS = {"verify.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _run(cmd: list[str]) -> None:
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


HIP_SOURCES = ["flare_hip.hip", "mvs_q8_0.hip", "mvs_q4k.hip", "mvs_f32.hip", "attn.hip", "verify.hip", "mvo.hip", "seq.hip",
               "sample.hip", "fused.hip"]
HOST_SOURCES = ["synth.cpp", "generate.cpp", "gguf.cpp"]


def build(verbose: bool = True) -> str:
    # FLARE_BUILD_DEFS: extra -D flags for diagnostic builds (e.g. -DFLARE_ATTN_TRACE)
    extra = os.environ.get("FLARE_BUILD_DEFS", "").split()
    from concurrent.futures import ThreadPoolExecutor

    os.makedirs(BUILD, exist_ok=True)
    jobs = []
    objs = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        jobs.append([HIPCC, *HIP_FLAGS, *SOURCE_FLAGS.get(src, []), *extra, "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    for src in HOST_SOURCES:
        obj = os.path.join(BUILD, src.replace(".cpp", ".o"))
        jobs.append(["g++", *CXX_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    workers = max(1, min(len(jobs), os.cpu_count() or 1, 8))
    with ThreadPoolExecutor(workers) as ex:
        for f in [ex.submit(_run, j) for j in jobs]:
            f.result()
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-lgomp", "-o", tmp])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
