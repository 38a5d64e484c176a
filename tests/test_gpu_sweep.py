"""A seeded random sweep of the parity tests over the space the fixed cases sample: single reads (list layout) of
random batch, token count, width, source count and position (boundary or not), fp32 and bf16, to the same bars as
tests/test_gpu_read.py; and small random chains (every layout and score mode) to the bars of tests/test_gpu_stack.py.
A second sweep draws from the whole input space -- any width (also not a multiple of 8, and above 8192), up to 96
sources, fp32, bf16 and fp16 -- for reads and chains alike (the any-shape kernels where the row-layout ones do not
take the call). The cases are drawn once from fixed seeds, so every run tests the same ones."""
import random

import pytest
import torch

from gpu_helpers import err_max, err_norm, err_rms, lowp, make
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


ANY_WIDTHS = [1, 3, 7, 12, 36, 100, 248, 333, 1000, 2050, 4100, 8200]
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _any_read_cases(count=24, seed=4242):
    rnd = random.Random(seed)
    out = []
    for k in range(count):
        d = rnd.choice(ANY_WIDTHS)
        n = rnd.choice([2, 5, 17, 64, 65, 96])
        b = rnd.randint(1, 2)
        t = rnd.randint(1, max(2, min(600, (1 << 21) // (b * d * n))))
        out.append((b, t, d, n, rnd.random() < 0.5, DTYPES[k % 3], rnd.randrange(1 << 20)))
    return out


@pytest.mark.parametrize("b,t,d,n,boundary,dtype,seed", _any_read_cases())
def test_random_read_any_shape_matches_oracle(b, t, d, n, boundary, dtype, seed):
    """Reads over the whole input space: fp32 to max-abs 1e-5 x RMS of the exact read, or, where the reference read
    in fp32 is itself further off (rows of one to a few elements: the scale's gradient then cancels most of the
    update's), no more than twice its error; bf16 and fp16 no further from the exact read than the reference read in
    the same dtype (<= 2 err_ref + 2e-3, fp16 + 2.5e-4), and for rows of at least 8 elements what the kernels compute
    within max-abs 1e-2 x max|ref| (fp16 1.25e-3), the bars of test_16bit_against_fp64."""
    args = make(b, t, d, n, dtype, seed=seed)
    print(f"case any sweep read b{b} t{t} d{d} n{n} boundary={boundary} {dtype} seed={seed}", flush=True)
    hip = run_hip(d, n, args, boundary)
    ref64 = run_oracle(d, n, args, boundary, dtype=torch.float64)
    ref_dt = run_oracle(d, n, args, boundary)
    if dtype == torch.float32:
        e64, er = compare(hip, ref64, err_rms), compare(ref_dt, ref64, err_rms)
        assert all(e64[k] <= max(1e-5, 2 * er[k]) for k in e64), (e64, er)
        return
    ef = compare(hip, ref64, err_max)
    er = compare(ref_dt, ref64, err_max)
    if d >= 8:
        assert max(ef[k] for k in ("out", "tc", "dq", "dv", "dcoef")) <= lowp(1e-2, dtype), ef
    assert all(ef[k] <= 2 * er[k] + lowp(2e-3, dtype) for k in ef), (ef, er)


def _any_chain_cases(count=12, seed=99):
    rnd = random.Random(seed)
    out = []
    for k in range(count):
        K, R = rnd.randint(1, 4), rnd.randint(1, 5)
        if K * R < 2:
            R = 2
        d = rnd.choice(ANY_WIDTHS[1:])
        t = rnd.randint(1, max(2, min(200, (1 << 19) // (d * K * R))))
        out.append((K, R, d, t, ["list", "stack", "scores"][k % 3], DTYPES[(k // 3) % 3], [0.02, 0.5][(k // 2) % 2],
                    "0" if k % 2 else "1"))
    return out


@pytest.mark.parametrize("K,R,d,t,mode,dtype,q_std,glue", _any_chain_cases())
def test_random_chain_any_shape_matches_oracle(monkeypatch, K, R, d, t, mode, dtype, q_std, glue):
    """Random chains over any width and every dtype to the chain bars (check_chain). Query scales that leave the
    softmax unsaturated: with a saturated one a 16-bit chain is ill-conditioned (the bf16 reference chain itself ends
    1.5e-2 from the exact one, and single gradients up to 14 %), which test_chain_with_saturated_reads covers."""
    from loopback_amd.chain import ChainConfig
    from test_gpu_stack import check_chain, hip_chain
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", glue)
    cfg = ChainConfig(f"any-sweep-K{K}R{R}d{d}t{t}", d, K, R, 1, t, dtype, True, q_std=q_std)
    print(f"case any sweep chain K{K} R{R} d{d} t{t} {mode} {dtype} q_std={q_std} glue={glue}", flush=True)
    h, g = hip_chain(cfg, mode)
    check_chain(h, g, cfg)
