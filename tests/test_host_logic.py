"""Host-side logic that runs without a GPU: the drop-in's gates and errors, the stack's bookkeeping, the traffic
formula the bench reports against, and the bench's refusal of several GPUs."""
import os
import subprocess
import sys

import pytest
import torch

from loopback_amd import chain as C
from loopback_amd import fused_dattn as FD
from loopback_amd.cell import LoopDeltaAttnRes, stack_mode

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_interface_names():
    for name in ("rstd_ref", "rstd", "fused_read_supported", "FusedDattnRead", "DattnGradAccum", "FusedDattnReadAcc",
                 "DattnStack", "FusedDattnReadStk", "_alias"):
        assert hasattr(FD, name), name
    for attr in ("V", "R", "dV", "dR", "n_steps", "n_tok", "d", "eps", "Q", "QT", "DOTS", "r_done"):
        assert attr in FD.DattnStack.__slots__


def test_supported_is_false_on_cpu():
    v = [torch.randn(1, 4, 64) for _ in range(3)]
    r = [torch.ones(1, 4, 1) for _ in range(3)]
    assert FD.fused_read_supported(v[0].clone(), v, r, torch.ones(1, 4, 3)) is False


def test_rstd_on_cpu_tensors_is_rstd_ref():
    """Off the GPU, rstd returns rstd_ref, as the reference module does (fused_dattn.py:257-261): the same tensor
    bitwise; r x equals torch's own rms_norm (the library routine), and the gradient is the closed form
    gr (-r^3) x / d (fused_dattn.py:232-254), for every update dtype."""
    g = torch.Generator().manual_seed(5)
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        x = (torch.randn(2, 3, 64, generator=g) * 1.7).to(dtype).requires_grad_()
        r = FD.rstd(x, 1e-6)
        assert r.dtype == torch.float32 and r.shape == (2, 3, 1)
        assert torch.equal(r, FD.rstd_ref(x, 1e-6))
        xf = x.detach().double()
        rn = torch.nn.functional.rms_norm(xf, (64,), eps=1e-6)
        assert torch.allclose(r.double() * xf, rn, rtol=1e-6, atol=1e-6)
        gr = torch.randn(2, 3, 1, generator=g)
        r.backward(gr)
        r64 = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
        want = gr.double() * (-r64 ** 3) * xf / 64
        tol = {torch.float32: 1e-5, torch.bfloat16: 1e-2, torch.float16: 2e-3}[dtype]
        assert (x.grad.double() - want).abs().max().item() <= tol * want.abs().max().item()


def test_reference_combine_on_cpu_falls_back_to_its_read():
    """The reference cell with LOOP_DATTN_FUSED=1 on CPU tensors (looped_transformer.py:392-404): it caches
    `fused.rstd` of each update, asks `fused.fused_read_supported`, gets False and runs its own read. With this
    module as `fused` that sequence completes (rstd takes CPU tensors), the gate refuses every read, and the chain's
    final state and gradients are bitwise those of the reference read alone (the oracle's restatement of it; the
    fallback is the caller's read, never this module's)."""
    from oracle.reference_read import OracleCell
    K, R, d, T, eps, beta = 2, 2, 64, 6, 1e-6, 0.75
    g = torch.Generator().manual_seed(11)
    h0 = torch.randn(1, T, d, generator=g)
    D = [torch.randn(1, T, d, generator=g) for _ in range(K * R)]
    Q = torch.randn(K * R - 1, d, generator=g) * 0.5
    G = torch.randn(1, T, d, generator=g)
    refused = []

    def combine(cell, proposal, h0_, deltas, coeffs, prior, l, blk, keys):
        # the fused branch of the reference cell, with this module as `fused`
        step = l * K + blk
        at_end = blk == K - 1
        base = proposal + beta * (h0_ - proposal) if at_end else proposal
        one = torch.ones(*proposal.shape[:-1], 1)
        base_coeffs = one if coeffs is None else torch.cat((coeffs, one), -1)
        if at_end:
            base_coeffs = (1 - beta) * base_coeffs
        if len(keys) < len(deltas):
            keys.append(FD.rstd(deltas[-1], eps))
        if len(deltas) > 1:
            ok = FD.fused_read_supported(base, deltas, keys, base_coeffs)
            refused.append(not ok)
            assert step >= 1
        return cell.combine(proposal, h0_, deltas, coeffs, prior, l, blk, keys=None)

    def run(via_module):
        q = Q.clone().requires_grad_()
        h0_ = h0.clone().requires_grad_()
        Dl = [x.clone().requires_grad_() for x in D]
        cell = OracleCell(d, R, K, beta, eps, q)
        h, deltas, keys, coeffs, prior = h0_, [], [], None, None
        for s in range(K * R):
            l, blk = divmod(s, K)
            x = h
            hs = x + Dl[s]
            deltas.append(hs - x)
            if via_module:
                h, coeffs, prior = combine(cell, hs, h0_, deltas, coeffs, prior, l, blk, keys)
            else:
                h, coeffs, prior = cell.combine(hs, h0_, deltas, coeffs, prior, l, blk)
        (h * G).sum().backward()
        return [h.detach(), h0_.grad, q.grad] + [x.grad for x in Dl]

    got = run(True)
    assert refused == [True] * (K * R - 1)
    for a, b in zip(got, run(False)):
        assert torch.equal(a, b)


def test_stack_refuses_cpu_and_bad_shapes():
    """Any width >= 1 and up to ANY_MAX_SOURCES steps are shapes the stack takes (on a GPU); a CPU device, no
    width, no steps or more steps than the kernels take are refused."""
    with pytest.raises(RuntimeError, match="GPU"):
        FD.DattnStack(4, (1, 8, 64), torch.bfloat16, "cpu")
    with pytest.raises(RuntimeError, match="GPU"):
        FD.DattnStack(70, (1, 8, 60), torch.bfloat16, "cpu")
    for steps, d in ((4, 0), (0, 64), (FD.ANY_MAX_SOURCES + 1, 64)):
        with pytest.raises(RuntimeError, match="unsupported shape"):
            FD.DattnStack(steps, (1, 8, d), torch.bfloat16, "cpu")


def test_pair_rows_cover_the_triangle():
    N = 32
    rows = [FD._pair(s, i) for s in range(1, N) for i in range(s + 1)]
    assert rows == list(range(N * (N + 1) // 2 - 1))


def test_cell_validation_errors():
    cell = LoopDeltaAttnRes(64, 2, 3)
    assert tuple(cell.query.shape) == (5, 64) and torch.count_nonzero(cell.query) == 0
    x = torch.zeros(1, 2, 64)
    with pytest.raises(ValueError):
        cell.combine(x, x, [x], None, None, 0, 3)
    with pytest.raises(ValueError):
        cell.combine(x, x, [x], None, None, 2, 0)
    with pytest.raises(ValueError):
        cell.combine(x, x, [x, x], None, None, 0, 0)
    with pytest.raises(ValueError):
        LoopDeltaAttnRes(64, 0, 3)
    with pytest.raises(ValueError):
        LoopDeltaAttnRes(64, 2, 3, beta=1.0)


def test_mode_flags(monkeypatch):
    monkeypatch.setenv("LOOP_DATTN_STACK", "1")
    monkeypatch.setenv("LOOP_DATTN_DOTS", "1")
    assert stack_mode() == "scores"
    monkeypatch.setenv("LOOP_DATTN_DOTS", "0")
    assert stack_mode() == "stack"
    monkeypatch.setenv("LOOP_DATTN_STACK", "0")
    assert stack_mode() == "list"


def test_traffic_formula_of_the_reference_dataflow():
    # headline: d=2048, N=32, bf16: e d (5N + 4 S2 + 4(N-1)) = 4096 * 2392 = 9,797,632 bulk bytes per token
    parts = C.algorithmic_bytes_per_token(32, 2048, 2)
    assert parts["total"] == 9_797_632
    assert C.algorithmic_bytes_per_token(8, 768, 2, backward=False)["total"] == (3 * 8 + 35 + 14) * 768 * 2


def test_per_kernel_bytes_add_up_to_the_formula():
    """The bench's per-family byte models: the reference dataflow's rows per family sum to the whole-pass formula,
    and this build's own rows differ from them only by its documented extras (the fused blend's h0 rows, the
    update gradient's own rows in place of the read-modify-written gradient stack)."""
    sys.path.insert(0, ROOT)
    import bench
    for name in ("c2", "c3", "c4"):
        cfg = C.CONFIGS[name]
        ref, extra = bench.reference_bytes(cfg, "scores")
        fam, ref_total = bench.family_bytes(cfg, "scores")
        assert sum(ref.values()) == ref_total, name
        row = cfg.d * torch.empty(0, dtype=cfg.dtype).element_size() * cfg.n_tok
        assert fam["read_fwd"] - ref["read_fwd"] == extra["read_fwd"] * row, name   # h0 at each iteration end
        assert fam["write_dots"] == ref["write_dots"] and fam.get("read_bwd1") == ref.get("read_bwd1"), name


def test_configs():
    c4 = C.CONFIGS["c4"]
    assert (c4.d, c4.N, c4.n_tok, c4.dtype, c4.backward) == (2048, 32, 16384, torch.bfloat16, True)
    assert C.CONFIGS["c1"].n_tok == 512 and C.CONFIGS["c3"].N == 12


def test_bench_refuses_several_gpus():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                         text=True, timeout=120)
    assert res.returncode != 0
    assert "one GPU" in (res.stdout + res.stderr)


def test_remap_query_rows():
    """Extra iterations at evaluation: trained reads keep their rows; a new read takes the row of the same block
    position in the last trained iteration ('last') or a zero row ('zero'); R below the trained count truncates."""
    import torch
    from loopback_amd.cell import remap_query
    K, R0 = 4, 2
    q = torch.arange((K * R0 - 1) * 3, dtype=torch.float32).view(K * R0 - 1, 3)
    last = remap_query(q, K, R0, 4, "last")
    zero = remap_query(q, K, R0, 4, "zero")
    assert last.shape == zero.shape == (K * 4 - 1, 3)
    assert torch.equal(last[:K * R0 - 1], q) and torch.equal(zero[:K * R0 - 1], q)
    for s in range(K * R0, K * 4):                      # destination read s uses row s - 1
        assert torch.equal(last[s - 1], q[(R0 - 1) * K + s % K - 1])
        assert not zero[s - 1].any()
    # K = 1: the first new read's source row is the last trained read (row R0 - 1 - 1 + 0)
    q1 = torch.randn(2, 5)
    r1 = remap_query(q1, 1, 3, 5, "last")
    assert torch.equal(r1[2], q1[1]) and torch.equal(r1[3], q1[1])
    assert torch.equal(remap_query(q, K, R0, 1, "last"), q[:K - 1])
    with pytest.raises(ValueError):
        remap_query(q, K, R0, 4, "first")


def test_build_defines(monkeypatch):
    """The launch settings a build takes (the counterpart of the reference module's tunable launch globals):
    LDR_NAME=VALUE words from -D and from LOOPBACK_READ_DEFINES, nothing else."""
    from loopback_amd.build import _defines
    monkeypatch.delenv("LOOPBACK_READ_DEFINES", raising=False)
    assert _defines(["LDR_RF_GRID=768"]) == ["-DLDR_RF_GRID=768"]
    monkeypatch.setenv("LOOPBACK_READ_DEFINES", "LDR_B1_TT=16 LDR_NT=0")
    assert _defines([]) == ["-DLDR_B1_TT=16", "-DLDR_NT=0"]
    for bad in (["RF_GRID=1"], ["LDR_X=1; rm"], ["-O0"]):
        with pytest.raises(ValueError):
            _defines(bad)


def test_missing_library_fails_at_import():
    """No CPU fallback: without the built library the drop-in module does not import (the reference's callers then
    take their own read, as for any import failure, looped_transformer.py:325-330)."""
    env = dict(os.environ, LOOPBACK_READ_LIB=os.path.join(ROOT, "_no_such_dir", "libloopback_read.so"))
    proc = subprocess.run([sys.executable, "-c", "import loopback_amd.fused_dattn"], cwd=ROOT, env=env,
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode != 0
    assert "ImportError" in proc.stderr and "no fallback" in proc.stderr, proc.stderr[-2000:]
