"""Build libbrx.so (the HIP kernels and C-ABI) for gfx950, in-tree, with hipcc, and the
host-only trace-replay library libbrx_replay.so with g++.

    python -m bigrig_amd.build            # compile bigrig_amd/libbrx.so and libbrx_replay.so
    python -m bigrig_amd.build --incremental   # recompile only sources changed since their object

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


def _run(cmd, verbose: bool, what: str) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"{what} failed ({r.returncode}):\n{out}")
    if verbose and out.strip():
        print(out)


def build(verbose: bool = False, incremental: bool = False) -> str:
    """Compile every csrc/*.hip to an object in parallel (each file carries its own device code
    object; kernels are only launched from the file that defines them), then link. With
    `incremental`, objects newer than their source and every header are kept."""
    from concurrent.futures import ThreadPoolExecutor
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objdir = os.path.join(PKG, "_build")
    os.makedirs(objdir, exist_ok=True)
    flags = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-mllvm", "-amdgpu-mfma-vgpr-form=1",
             "-Wno-unused-command-line-argument", "-I", INCLUDE, "-I", CSRC]
    objs = [os.path.join(objdir, os.path.basename(s)[:-4] + ".o") for s in srcs]
    headers = glob.glob(os.path.join(CSRC, "*.h")) + glob.glob(os.path.join(INCLUDE, "*.h"))
    newest_h = max((os.path.getmtime(h) for h in headers), default=0.0)

    def stale(s, o):
        return (not incremental or not os.path.exists(o) or
                os.path.getmtime(o) < max(os.path.getmtime(s), newest_h))

    jobs = min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(_run, [hipcc(), *flags, "-c", s, "-o", o], verbose, f"hipcc {s}")
                for s, o in zip(srcs, objs) if stale(s, o)]
        for f in futs:
            f.result()
    tmp = LIB + ".tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp], verbose,
         "hipcc link")
    os.replace(tmp, LIB)
    build_replay(verbose)
    return LIB


def build_replay(verbose: bool = False) -> str:
    """libbrx_replay.so: csrc/replay.cpp, plain C++ for the host (no GPU code)."""
    tmp = REPLAY_LIB + ".tmp"
    # -ffp-contract=off: the floating-point policies (LFUDA, gaterank, coact) must round each
    # step as the Python restatement does, so their victims agree request for request
    cmd = [shutil.which("g++") or "g++", "-O3", "-std=c++17", "-ffp-contract=off", "-fPIC",
           "-shared", "-pthread",
           "-I", INCLUDE, os.path.join(CSRC, "replay.cpp"), "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed ({r.returncode}):\n{r.stdout}{r.stderr}")
    os.replace(tmp, REPLAY_LIB)
    return REPLAY_LIB


if __name__ == "__main__":
    print(build(verbose="-q" not in sys.argv, incremental="--incremental" in sys.argv))
