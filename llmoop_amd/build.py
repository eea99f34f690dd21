"""Builds llmoop_amd/libnerve_sampler.so for gfx950 with hipcc.

Flags that the sampler's bit-exactness depends on:
  -ffp-contract=off                     no fused multiply-add: one rounding per op
  -fno-gpu-flush-denormals-to-zero      binary32 subnormals kept, as on the host
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed fp32 instructions
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libnerve_sampler.so")
SOURCES = ["nerve_sampler_kernels.hip", "nerve_sampler_api.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-I", os.path.join(ROOT, "include"),
    "-I", CSRC,
]


def build(verbose: bool = False) -> str:
    cmd = [HIPCC, *FLAGS, "-x", "hip", *[os.path.join(CSRC, s) for s in SOURCES], "-o", LIB]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed building libnerve_sampler.so")
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
