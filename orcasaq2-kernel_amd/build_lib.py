"""Builds libexl3hip.so (the gfx950 HIP kernels + C ABI) into the orcasaq2 package.

    python orcasaq2-kernel_amd/build_lib.py [-v]

Each csrc/*.hip file is compiled on its own (in parallel) with hipcc for gfx950, then
linked into orcasaq2/libexl3hip.so.  Cross-compiles without a GPU.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "orcasaq2", "libexl3hip.so")
MEASURE = os.path.join(CSRC, "measure")
CEILING = os.path.join(HERE, "orcasaq2", "libexl3ceiling.so")
REPLAY_SRC = os.path.join(CSRC, "replay", "addr_replay.hip")
REPLAY = os.path.join(HERE, "orcasaq2", "libexl3replay.so")
ARCH = os.environ.get("EXL3_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall",
    "-Wno-unused-function",
    # packed fp32 VALU forms are kept off for all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", CSRC, "-I", INCLUDE,
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libexl3hip)")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def build(verbose: bool = False, jobs: int | None = None) -> str:
    os.makedirs(BUILD, exist_ok=True)
    cc = hipcc()
    srcs = sources()
    objs = [os.path.join(BUILD, os.path.basename(s)[:-4] + ".o") for s in srcs]

    def compile_one(src_obj):
        src, obj = src_obj
        cmd = [cc] + HIPCC_FLAGS + ["-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed for {os.path.basename(src)}:\n{r.stdout}\n{r.stderr}")
        return r.stderr

    jobs = jobs or min(8, os.cpu_count() or 4, len(srcs))
    with cf.ThreadPoolExecutor(jobs) as ex:
        for warn in ex.map(compile_one, zip(srcs, objs)):
            if verbose and warn.strip():
                print(warn, file=sys.stderr)
    tmp = OUT + ".tmp"
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, OUT)
    build_ceiling(verbose)
    build_replay(verbose)
    return OUT


def build_ceiling(verbose: bool = False) -> str:
    """The measurement library of bench.py --workload ceiling (csrc/measure/*.hip): kernels
    that walk a shard the way the batch-1 GEMV does but stop short of parts of its work, and
    instruction-rate chains.  Not part of libexl3hip or its C ABI."""
    cc = hipcc()
    srcs = sorted(os.path.join(MEASURE, f) for f in os.listdir(MEASURE) if f.endswith(".hip"))
    tmp = CEILING + ".tmp"
    cmd = [cc] + HIPCC_FLAGS + ["-shared", "-o", tmp] + srcs
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for the measurement library:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, CEILING)
    return CEILING


def build_replay(verbose: bool = False) -> str:
    """The CPU address replay of the GEMV and stream-K GEMM plans (csrc/replay): host code
    only, checked by the CPU test suite.  Not part of libexl3hip or its C ABI."""
    cc = hipcc()
    tmp = REPLAY + ".tmp"
    cmd = [cc] + HIPCC_FLAGS + ["-shared", "-o", tmp, REPLAY_SRC]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for the address replay:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, REPLAY)
    return REPLAY


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
