"""Builds libnumrs_hip.so (the HIP backend) in-tree with hipcc for gfx950.

    python -m numrs_amd.build          # or numrs_amd.build.build()

Each .hip source compiles separately (in parallel) and links into
numrs_amd/lib/libnumrs_hip.so.  Flags:
  --offload-arch=gfx950                 the only target
  -ffp-contract=off                     never fuse a*b+c (the reference does not)
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                        no packed-fp32 VALU instructions
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJ = os.path.join(PKG, "lib", "obj")
LIB = os.path.join(PKG, "lib", "libnumrs_hip.so")

SOURCES = ["runtime.hip", "gemm.hip", "eltwise.hip", "reduce.hip", "rowwise.hip", "fwd.hip",
           "attention.hip", "lstm.hip", "optim.hip", "dispatch.hip", "autograd.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{proc.stderr[-4000:]}")
    # hipcc's host pass does not know the packed-fp32 feature; that warning is expected.
    return obj


def build(verbose: bool = False) -> str:
    """Compiles every HIP source and links the shared library; returns its path."""
    if not os.path.exists(HIPCC) and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found; cannot build the HIP backend")
    os.makedirs(OBJ, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as pool:
        objs = list(pool.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr[-4000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
