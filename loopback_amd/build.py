"""Build libloopback_read.so (the read's kernels and C ABI) in-tree with hipcc for gfx950 (MI355X).

    python -m loopback_amd.build                          # compile, print the commands
    python -m loopback_amd.build -D LDR_RF_GRID=768 ...   # with launch settings other than the measured defaults
    python -m loopback_amd.build -D LDR_WRITE_VALU=1 --out /path/lib.so   # a comparison build of the library alone

The launch settings (the LDR_* constants at the top of csrc/loopback_read.hip: sources per batch, workgroups,
tile sizes, staging space) are compile-time constants of the kernels; -D NAME=VALUE (or LOOPBACK_READ_DEFINES,
space-separated NAME=VALUE words) sets them for a build -- the counterpart of the reference module's tunable launch
globals (fused_dattn.py:43-52). The libraries land next to this file, so they travel with the source tree to the GPU
box; nothing is installed. Compiling needs hipcc only, not a GPU.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "csrc", "loopback_read.hip")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(HERE, "libloopback_read.so")
# A test fixture: the same source built with the alternative kernel shapes -- the write in the matrix cores' layout
# for every width and dtype (LDR_WM_ROWS=0, LDR_W32_ROWS=0), the read forward in 256-lane workgroups for every read
# (LDR_RF_BIG=0) -- so the
# GPU tests can check that the shapes the product library picks give the same bits. Nothing else loads it.
TEST_LIB_ALT = os.path.join(HERE, "libloopback_read_alt_shapes.so")
ALT_DEFINES = ["LDR_WM_ROWS=0", "LDR_W32_ROWS=0", "LDR_RF_BIG=0"]
# A test program: the C ABI used from C alone (tests/c_abi/abi_smoke.c), linked against the product library.
ABI_SMOKE_SRC = os.path.join(ROOT, "tests", "c_abi", "abi_smoke.c")
ABI_SMOKE = os.path.join(ROOT, "tests", "c_abi", "abi_smoke")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in the generated code (plain fp32 VALU instead).
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the loopback_read library cannot be built")
    return path


_DEFINE = re.compile(r"LDR_[A-Z0-9_]+(=[A-Za-z0-9_.+-]+)?")


def _defines(defines) -> list[str]:
    words = list(defines or []) + os.environ.get("LOOPBACK_READ_DEFINES", "").split()
    for w in words:
        if not _DEFINE.fullmatch(w):
            raise ValueError(f"loopback_read build: a define must be LDR_NAME[=VALUE], got {w!r}")
    return [f"-D{w}" for w in words]


def _start(src: str, lib: str, verbose: bool, defines) -> tuple:
    tmp = lib + ".tmp"
    cmd = [hipcc(), *FLAGS, *_defines(defines), f"-I{INCLUDE}", "-o", tmp, src]
    if verbose:
        print(" ".join(cmd), flush=True)
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True), tmp, lib


def _wait(job) -> str | None:
    """Wait for one compile; install its output, or return its error message."""
    proc, tmp, lib = job
    out, err = proc.communicate()
    if proc.returncode != 0:
        return f"hipcc failed ({proc.returncode}) for {os.path.basename(lib)}:\n{out}\n{err}"
    os.replace(tmp, lib)
    return None


def _finish(job) -> None:
    msg = _wait(job)
    if msg is not None:
        raise RuntimeError(msg)


def build_abi_smoke(verbose: bool = True) -> str:
    """Compile the C test program against include/ and the built library (gcc, the HIP runtime's C API)."""
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("no C compiler: the C ABI test program cannot be built")
    tmp = ABI_SMOKE + ".tmp"
    cmd = [cc, "-std=c11", "-O2", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include",
           f"-I{INCLUDE}", ABI_SMOKE_SRC, f"-L{ROCM}/lib", "-lamdhip64", f"-L{HERE}", "-lloopback_read",
           "-Wl,-rpath,$ORIGIN/../../loopback_amd", f"-Wl,-rpath,{ROCM}/lib", "-lm", "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"the C ABI test program failed to build ({proc.returncode}):\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, ABI_SMOKE)
    return ABI_SMOKE


def build(verbose: bool = True, defines=None, fixtures: bool = True) -> str:
    """Compile the library (always; a stale build never survives a call) and, with `fixtures`, beside it the test
    fixture TEST_LIB_ALT (the two compiles run in parallel) and then the C ABI test program; returns the library's
    path. Every compile started is waited for before any error is raised. The library's failure raises; a test
    fixture's is reported on stderr and does not fail the library's build (the GPU tests that load the fixture then
    fail on its absence). defines: NAME=VALUE launch settings (see the module docstring)."""
    jobs = [_start(SRC, LIB, verbose, defines)]
    if fixtures:
        jobs.append(_start(SRC, TEST_LIB_ALT, verbose, list(defines or []) + ALT_DEFINES))
    errors = [_wait(job) for job in jobs]
    if errors[0] is not None:
        raise RuntimeError(errors[0])
    fixture_errors = [e for e in errors[1:] if e is not None]
    if fixtures and not fixture_errors:
        try:
            build_abi_smoke(verbose)
        except RuntimeError as e:
            fixture_errors.append(str(e))
    for e in fixture_errors:
        print(f"loopback_read build: a test fixture was not built (the library was): {e}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    import argparse
    ap = argparse.ArgumentParser(description="build the loopback_read library for gfx950")
    ap.add_argument("-D", dest="defines", action="append", default=[], metavar="LDR_NAME=VALUE",
                    help="a launch setting of the read kernels (repeatable)")
    ap.add_argument("--out", default=None, metavar="PATH",
                    help="build only the library, to PATH (a comparison build, loaded with LOOPBACK_READ_LIB=PATH)")
    args = ap.parse_args()
    if args.out:
        _finish(_start(SRC, os.path.abspath(args.out), True, args.defines))
    else:
        build(defines=args.defines)
    sys.exit(0)
