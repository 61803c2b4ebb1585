"""Build libbrx.so (the HIP kernels and C-ABI) for gfx950, in-tree, with hipcc, and the
host-only trace-replay library libbrx_replay.so with g++.

    python -m bigrig_amd.build            # compile bigrig_amd/libbrx.so and libbrx_replay.so

The library is one hipcc invocation over every `csrc/*.hip` file. Packed FP32 instructions are
disabled for device code (`-Xclang -target-feature -Xclang -packed-fp32-ops`); the host pass
warns that it does not know that feature, which is harmless. MFMA accumulators are allocated in
ordinary VGPRs (`-mllvm -amdgpu-mfma-vgpr-form=1`): with them in AGPRs the register allocator
rotated the prefill GEMM's accumulators between loop iterations, costing ~190 register copies
per K step.
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(PKG, "libbrx.so")
REPLAY_LIB = os.path.join(PKG, "libbrx_replay.so")
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build libbrx")


def build(verbose: bool = False) -> str:
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-mllvm", "-amdgpu-mfma-vgpr-form=1",
           "-Wno-unused-command-line-argument", "-I", INCLUDE, "-I", CSRC,
           *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{out}")
    if verbose and out.strip():
        print(out)
    os.replace(tmp, LIB)
    build_replay(verbose)
    return LIB


def build_replay(verbose: bool = False) -> str:
    """libbrx_replay.so: csrc/replay.cpp, plain C++ for the host (no GPU code)."""
    tmp = REPLAY_LIB + ".tmp"
    cmd = [shutil.which("g++") or "g++", "-O3", "-std=c++17", "-fPIC", "-shared", "-pthread",
           "-I", INCLUDE, os.path.join(CSRC, "replay.cpp"), "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed ({r.returncode}):\n{r.stdout}{r.stderr}")
    os.replace(tmp, REPLAY_LIB)
    return REPLAY_LIB


if __name__ == "__main__":
    print(build(verbose="-q" not in sys.argv))
