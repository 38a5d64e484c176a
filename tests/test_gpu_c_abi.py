"""The C ABI from C alone: tests/c_abi/abi_smoke (built by loopback_amd.build against include/loopback_read.h and the
product library) allocates with hipMalloc and calls the entry points with no Python or torch in the process: the
scale and its gradient, the online and stored-score reads and the any-shape read, backward pass 1 with and without
a workspace, the list layout's pass 2 and the stacked assembly, the fp32 and bf16 writes, the blends' sum and the
argument errors, each checked against a closed form, an identity, another entry point or a dot product (the
program's header lists them). It runs as a child process."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu


def test_c_program_uses_the_abi():
    from loopback_amd import build as B
    if not os.path.exists(B.ABI_SMOKE):
        raise RuntimeError(f"{B.ABI_SMOKE} is not built (run `python -m loopback_amd.build`)")
    print("case C ABI program", flush=True)
    proc = subprocess.run([B.ABI_SMOKE], capture_output=True, text=True, timeout=120)
    print(proc.stdout, flush=True)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "abi smoke: ok" in proc.stdout, proc.stdout
