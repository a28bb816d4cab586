"""Builds the native library of the package in-tree.

`build()` compiles every HIP source for gfx950 and the host C++ runtime into
tinyinfer_amd/lib/libminiprefix_hip.so with hipcc, then the protocol-v3
worker executable tinyinfer_amd/lib/miniprefix_worker against it. There is
no CPU fallback: the Python side refuses to run without this library.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
LIB_DIR = PACKAGE / "lib"
LIBRARY = LIB_DIR / "libminiprefix_hip.so"
WORKER = LIB_DIR / "miniprefix_worker"

ARCH = os.environ.get("MP_HIP_ARCH", "gfx950")

# -ffp-contract=off keeps the reference's separate multiply/add roundings;
# packed FP32 instructions are disabled on purpose.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def sources() -> list[Path]:
    hip = sorted((CSRC / "backend").glob("*.hip"))
    host = sorted((CSRC / "host").glob("*.cpp")) if (CSRC / "host").exists() else []
    return hip + host


def build(verbose: bool = False) -> Path:
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc, *HIP_FLAGS, "-shared", "-o", str(tmp),
           f"-I{ROOT / 'include'}", f"-I{CSRC / 'host'}", f"-I{CSRC / 'backend'}",
           *[str(s) for s in sources()]]
    if verbose:
        print(" ".join(cmd), file=sys.stderr)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l and "(ignoring feature)" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIBRARY)
    build_worker(verbose)
    return LIBRARY


def build_worker(verbose: bool = False) -> Path:
    """The worker executable (csrc/worker), linked to the library beside it."""
    worker = CSRC / "worker"
    tmp = WORKER.with_suffix(".tmp")
    cmd = [os.environ.get("CXX", "g++"), "-std=c++17", "-O2", "-Wall", f"-I{ROOT / 'include'}",
           f"-I{CSRC / 'host'}", f"-I{worker}", str(worker / "worker.cpp"), str(worker / "protocol.cpp"),
           f"-L{LIB_DIR}", "-lminiprefix_hip", "-Wl,-rpath,$ORIGIN", "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), file=sys.stderr)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"worker build failed ({proc.returncode}):\n{proc.stderr[-4000:]}")
    os.replace(tmp, WORKER)
    return WORKER


if __name__ == "__main__":
    print(build(verbose=True))
