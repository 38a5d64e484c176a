"""Build libloopback_read.so in-tree with hipcc for gfx950 (MI355X).

    python -m loopback_amd.build            # compile, print the command

The library lands next to this file (loopback_amd/libloopback_read.so), so it travels with the source tree to the
GPU box; nothing is installed. Compiling needs hipcc only, not a GPU.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "csrc", "loopback_read.hip")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(HERE, "libloopback_read.so")
ARCH = "gfx950"

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in the generated code (plain fp32 VALU instead).
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the loopback_read library cannot be built")
    return path


def build(verbose: bool = True) -> str:
    """Compile the library (always; a stale build never survives a call) and return its path."""
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *FLAGS, f"-I{INCLUDE}", "-o", tmp, SRC]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
