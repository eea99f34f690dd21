"""Builds llmoop_amd/libnerve_sampler.so for gfx950 with hipcc.

Each source compiles to its own object in parallel (the slice kernels are
split into one translation unit per variant), then hipcc links the library.

Flags that the sampler's bit-exactness depends on:
  -ffp-contract=off                     no fused multiply-add: one rounding per op
  -fno-gpu-flush-denormals-to-zero      binary32 subnormals kept, as on the host
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed fp32 instructions
"""
from __future__ import annotations

import glob
import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libnerve_sampler.so")
OBJDIR = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-I", os.path.join(ROOT, "include"),
    "-I", CSRC,
]


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip"))) + [os.path.join(CSRC, "nerve_sampler_api.cpp")]


def _run(cmd: list[str], verbose: bool) -> str:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed: {' '.join(cmd[-3:])}")
    return res.stderr


def scratch_users(remarks: str) -> list[str]:
    """Kernels whose resource-usage remarks report private (scratch) memory:
    a spill or a dynamically indexed local array, which the sampling kernels
    must never have."""
    users, name = [], None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and name and int(m.group(1)) > 0:
            users.append(f"{name} ({m.group(1)} bytes/lane)")
    return users


def build(verbose: bool = False, jobs: int | None = None) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(OBJDIR, os.path.basename(s) + ".o") for s in srcs]
    cmds = [[HIPCC, *FLAGS, "-Rpass-analysis=kernel-resource-usage", "-x", "hip", "-c", s, "-o", o]
            for s, o in zip(srcs, objs)]
    workers = jobs or min(len(cmds), max(1, min(os.cpu_count() or 1, 16)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        remarks = list(pool.map(lambda c: _run(c, verbose), cmds))
    bad = scratch_users("\n".join(remarks))
    if bad:
        raise RuntimeError("kernels using scratch memory:\n  " + "\n  ".join(bad))
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", LIB], verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
