"""A seeded random sweep of the parity tests over the space the fixed cases sample: single reads (list layout) of
random batch, token count, width, source count and position (boundary or not), fp32 and bf16, to the same bars as
tests/test_gpu_read.py; and small random chains (every layout and score mode) to the bars of tests/test_gpu_stack.py.
The cases are drawn once from a fixed seed, so every run tests the same ones."""
import random

import pytest
import torch

from gpu_helpers import err_max, err_norm, err_rms, make
from test_gpu_read import compare, run_hip, run_oracle

pytestmark = pytest.mark.gpu

WIDTHS = [8, 16, 40, 64, 128, 264, 512, 768, 1000, 1024, 1536, 2048, 2056, 3072, 4096]


def _read_cases(count=28, seed=2026):
    rnd = random.Random(seed)
    out = []
    for k in range(count):
        d = rnd.choice(WIDTHS)
        n = rnd.randint(2, 40)
        b = rnd.randint(1, 3)
        t = rnd.randint(1, max(2, (1 << 22) // (b * d * n)))   # at most ~4M update elements per case
        out.append((b, t, d, n, rnd.random() < 0.5,
                    torch.float32 if k % 2 == 0 else torch.bfloat16, rnd.randrange(1 << 20)))
    return out


@pytest.mark.parametrize("b,t,d,n,boundary,dtype,seed", _read_cases())
def test_random_read_matches_oracle(b, t, d, n, boundary, dtype, seed):
    args = make(b, t, d, n, dtype, seed=seed)
    print(f"case sweep read b{b} t{t} d{d} n{n} boundary={boundary} {dtype} seed={seed}", flush=True)
    hip = run_hip(d, n, args, boundary)
    ref64 = run_oracle(d, n, args, boundary, dtype=torch.float64)
    if dtype == torch.float32:
        e64 = compare(hip, ref64, err_rms)
        assert max(e64.values()) <= 1e-5, e64
        return
    ef = compare(hip, ref64, err_max)
    er = compare(run_oracle(d, n, args, boundary), ref64, err_max)
    assert max(ef[k] for k in ("out", "tc", "dq", "dv", "dcoef")) <= 1e-2, ef
    assert all(ef[k] <= 2 * er[k] + 2e-3 for k in ef), (ef, er)


def _chain_cases(count=12, seed=77):
    rnd = random.Random(seed)
    out = []
    for k in range(count):
        K, R = rnd.randint(1, 4), rnd.randint(1, 4)
        if K * R < 2:
            R = 2
        out.append((K, R, rnd.choice([64, 264, 768, 1024, 2048]), rnd.randint(1, 300),
                    ["list", "stack", "scores"][k % 3], torch.float32 if k % 2 == 0 else torch.bfloat16,
                    rnd.choice([0.02, 0.5, 3.0]), "0" if k % 4 >= 2 else "1"))
    return out


@pytest.mark.parametrize("K,R,d,t,mode,dtype,q_std,glue", _chain_cases())
def test_random_chain_matches_oracle(monkeypatch, K, R, d, t, mode, dtype, q_std, glue):
    """Random chains to the chain bars of tests/test_gpu_stack.py (check_chain): the stacked ones with the caller's
    glue as torch ops (glue "0") or inside the kernels ("1")."""
    from loopback_amd.chain import ChainConfig
    from test_gpu_stack import check_chain, hip_chain
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", glue)
    cfg = ChainConfig(f"sweep-K{K}R{R}d{d}t{t}", d, K, R, 1, t, dtype, True, q_std=q_std)
    print(f"case sweep chain K{K} R{R} d{d} t{t} {mode} {dtype} q_std={q_std} glue={glue}", flush=True)
    h, g = hip_chain(cfg, mode)
    check_chain(h, g, cfg)
