"""Build libloopback_read.so (the read's kernels and C ABI) and libloopback_probe.so (the streaming-ceiling probes of
stream_probe.py) in-tree with hipcc for gfx950 (MI355X).

    python -m loopback_amd.build            # compile, print the commands

The libraries land next to this file, so they travel with the source tree to the GPU box; nothing is installed.
Compiling needs hipcc only, not a GPU.
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
PROBE_SRC = os.path.join(HERE, "csrc", "stream_probe.hip")
PROBE_LIB = os.path.join(HERE, "libloopback_probe.so")
ARCH = "gfx950"

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in the generated code (plain fp32 VALU instead).
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the loopback_read library cannot be built")
    return path


def _compile(src: str, lib: str, verbose: bool) -> None:
    tmp = lib + ".tmp"
    cmd = [hipcc(), *FLAGS, f"-I{INCLUDE}", "-o", tmp, src]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, lib)


def build(verbose: bool = True) -> str:
    """Compile both libraries (always; a stale build never survives a call); returns the read library's path."""
    _compile(SRC, LIB, verbose)
    _compile(PROBE_SRC, PROBE_LIB, verbose)
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
