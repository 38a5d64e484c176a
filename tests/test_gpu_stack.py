"""The stacked layout (DattnStack + FusedDattnReadStk, the trainer's default) and the list layout in K x R chains
against the oracle chain; mirrors tests/test_dattn_stack.py:68-199 of the reference.

  1. chains with blocks x -> x + D_s, every path ('list', 'stack' = stacked with online scores, 'scores' = stacked
     with scores stored at the write), the stacked paths both with the caller's glue as torch ops around
     FusedDattnReadStk (LOOP_DATTN_FUSE_GLUE=0: the reference trainer's own call sequence,
     modeling_looped_transformer.py:148-169) and inside the kernels (FusedCombineStk), fp32, bf16 and fp16 (the
     stack's dtype under fp16 mixed precision): the final state and the gradients of h0, every D_s and the query
     against the oracle chain in the same dtype (norm-relative 1e-5 in fp32, 1e-2 in bf16, 2.5e-3 in fp16; in fp32
     also max-abs <= 1e-5 x RMS against the exact (fp64) chain and against the fp32 chain); in bf16 and fp16 also
     no further from the fp64 oracle than the reference read itself is (<= 2 err_ref + 2e-3, fp16 + 2.5e-4). The
     list layout with in-kernel gradient accumulation (FusedDattnReadAcc) to the same bars, and bitwise the
     per-read gradients of the plain list layout;
     the stacked and list layouts' forwards are bitwise equal (the write stores the scale in the same summation
     order as the scale kernel), in training and in evaluation, fp32, bf16 and fp16;
  2. eval (no grad) chains, also with more iterations than trained (remapped queries);
  3. memory: a loss kept after its backward holds no stack;
  4. misuse: the reference module's RuntimeError cases and this build's limits;
  5. streams: a chain on a side stream, fwd+bwd, bitwise the default-stream chain;
  6. a NaN or inf in one token's input leaves every other token's result bitwise unchanged.
"""
import pytest
import torch

from gpu_helpers import DEV, err_max, err_norm, err_rms, lowp
from oracle.reference_read import run_chain as oracle_chain

pytestmark = pytest.mark.gpu


def chain_cfg(K, R, dtype, d=256, t=512, backward=True):
    from loopback_amd.chain import ChainConfig
    return ChainConfig(f"test-K{K}R{R}", d, K, R, 1, t, dtype, backward, q_std=0.5)


def hip_chain(cfg, mode, grad=True):
    from loopback_amd.chain import make_inputs, run_chain
    h0, D, Q, G = make_inputs(cfg, "cpu")
    h, loss, grads = run_chain(cfg, h0.to(DEV), [x.to(DEV) for x in D], Q.to(DEV), G.to(DEV), mode, grad=grad)
    torch.cuda.synchronize()
    return h.cpu(), grads


def ref_chain(cfg, dtype, grad=True):
    from loopback_amd.chain import make_inputs
    h0, D, Q, G = make_inputs(cfg, "cpu")
    if dtype == torch.float64:
        h0, D, Q, G = h0.double(), [x.double() for x in D], Q.double(), G.double()
    states, _, _, _, grads = oracle_chain(cfg.K, cfg.R, h0, D, Q, G, beta=cfg.beta, eps=cfg.eps, grad=grad)
    return states[-1], grads


def grad_list(g):
    return [g["h0"], g["query"]] + list(g["D"])


def check_chain(h, g, cfg, tol_fp32_rms=1e-5):
    """The chain bars against the oracle chain: norm-relative 1e-5 (fp32) / 1e-2 (bf16) / 2.5e-3 (fp16) against the
    oracle in the same dtype; fp32: max-abs <= 1e-5 x RMS against the exact (fp64) chain and the fp32 chain, for the
    final state and every gradient; bf16 and fp16: no further from the fp64 chain than the reference chain in the
    same dtype (<= 2 err_ref + 2e-3 in bf16, + 2.5e-4 in fp16, whose rounding is 8 times finer). The fp16 bar
    against the fp16 oracle is bf16's scaled by 1/4, not 1/8: the fp16 oracle chain itself is up to 1.3e-3 from the
    fp64 chain here."""
    hr, gr = ref_chain(cfg, None)
    h64, g64 = ref_chain(cfg, torch.float64)
    tol = {torch.float32: 1e-5, torch.bfloat16: 1e-2, torch.float16: 2.5e-3}[cfg.dtype]
    assert err_norm(h, hr) <= tol
    worst = max(err_norm(a, b) for a, b in zip(grad_list(g), grad_list(gr)))
    assert worst <= tol, worst
    if cfg.dtype == torch.float32:
        for ref_h, ref_g in ((h64, g64), (hr, gr)):
            e = [err_rms(h, ref_h)] + [err_rms(a, b) for a, b in zip(grad_list(g), grad_list(ref_g))]
            assert max(e) <= tol_fp32_rms, e
    else:
        slack = lowp(2e-3, cfg.dtype)
        assert err_norm(h, h64) <= 2 * err_norm(hr, h64) + slack
        for a, b, c in zip(grad_list(g), grad_list(gr), grad_list(g64)):
            assert err_norm(a, c) <= 2 * err_norm(b, c) + slack


@pytest.mark.parametrize("K,R", [(2, 4), (3, 3)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode,glue", [("list", "1"), ("stack", "1"), ("scores", "1"), ("stack", "0"),
                                       ("scores", "0")])
def test_chain_matches_oracle(monkeypatch, K, R, dtype, mode, glue):
    """glue "0": the stacked read as the reference trainer calls it (FusedDattnReadStk with the caller's torch glue,
    _RstdStk, _WriteDelta); "1": the glue inside the kernels (FusedCombineStk)."""
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", glue)
    cfg = chain_cfg(K, R, dtype)
    print(f"case chain K{K} R{R} {dtype} {mode} glue={glue}", flush=True)
    h, g = hip_chain(cfg, mode)
    check_chain(h, g, cfg)


@pytest.mark.parametrize("K,R,d,t", [(8, 8, 64, 33), (2, 2, 8192, 20), (1, 3, 8, 5), (2, 2, 64, 40001)])
@pytest.mark.parametrize("glue", ["1", "0"])
def test_stack_extremes_match_oracle(monkeypatch, K, R, d, t, glue):
    """The stacked layout at the row-layout kernels' limits in fp32: 64 steps (reads of up to 64 sources),
    the widest row, the narrowest row with one token per tile row, and a ragged 40001 tokens (several tiles per
    workgroup of the grid-capped kernels); glue as in test_chain_matches_oracle. Against the exact (fp64) chain:
    norm-relative and max-abs / RMS <= 1e-5, final state and every gradient."""
    from loopback_amd.chain import ChainConfig
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", glue)
    cfg = ChainConfig(f"edge-K{K}R{R}d{d}", d, K, R, 1, t, torch.float32, True, q_std=0.5)
    print(f"case stack edge K{K} R{R} d{d} t{t} glue={glue}", flush=True)
    for mode in ("scores", "stack"):
        h, g = hip_chain(cfg, mode)
        hr, gr = ref_chain(cfg, torch.float64)
        assert err_norm(h, hr) <= 1e-5
        worst = max(err_norm(a, b) for a, b in zip(grad_list(g), grad_list(gr)))
        assert worst <= 1e-5, (mode, worst)
        e = [err_rms(h, hr)] + [err_rms(a, b) for a, b in zip(grad_list(g), grad_list(gr))]
        assert max(e) <= 1e-5, (mode, e)


def list_chain(cfg, accumulate: bool, grad: bool = True):
    """The chain on the list layout with the caller's glue as torch ops (looped_transformer.py:380-403), each read
    through FusedDattnReadAcc (one DattnGradAccum per pass: the gradients accumulate in the kernels) or through
    FusedDattnRead (one gradient tensor per read and source, summed by autograd)."""
    from loopback_amd import fused_dattn as FD
    from loopback_amd.chain import make_inputs
    h0c, Dc, Q, G = make_inputs(cfg, "cpu")
    h0 = h0c.to(DEV).requires_grad_(grad)
    D = [x.to(DEV).requires_grad_(grad) for x in Dc]
    query = Q.to(DEV).requires_grad_(grad)
    acc = FD.DattnGradAccum()
    lam = 1.0 - cfg.beta
    with torch.set_grad_enabled(grad):
        h, deltas, keys, coeffs, prior = h0, [], [], None, None
        for s in range(cfg.N):
            blk = s % cfg.K
            x = h
            hs = x + D[s]
            deltas.append(hs - x)
            keys.append(FD.rstd(deltas[-1], cfg.eps))
            at_end = blk == cfg.K - 1
            base = hs + cfg.beta * (h0 - hs) if at_end else hs
            one = torch.ones(*hs.shape[:-1], 1, device=DEV)
            cb = one if coeffs is None else torch.cat((coeffs, one), -1)
            pr = torch.ones(1, device=DEV) if prior is None else torch.cat((prior, torch.ones(1, device=DEV)), -1)
            if at_end:
                cb, pr = lam * cb, lam * pr
            if s == 0:
                h, coeffs, prior = base, cb, pr
                continue
            if accumulate:
                h, coeffs = FD.FusedDattnReadAcc.apply(acc, s, query[s - 1], base, cb, pr, *deltas, *keys)
            else:
                h, coeffs = FD.FusedDattnRead.apply(query[s - 1], base, cb, pr, *deltas, *keys)
            prior = pr
        grads = None
        if grad:
            (h.float() * G.to(DEV)).sum().backward()
            torch.cuda.synchronize()
            grads = {"h0": h0.grad.cpu(), "query": query.grad.cpu(), "D": [x.grad.cpu() for x in D]}
    assert not acc.bufs or accumulate
    return h.detach().cpu(), grads


@pytest.mark.parametrize("K,R", [(2, 4), (3, 3), (1, 4)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_accumulating_list_chain_matches_oracle(K, R, dtype):
    """FusedDattnReadAcc (fused_dattn.py:337-376) in a chain: against the oracle chain to the chain bars, and every
    gradient bitwise the plain list layout's (FusedDattnRead, whose per-read gradients autograd adds): the kernel's
    accumulation prev + round(dv), rounded, is autograd's own bf16 add, in the same order (the reads' backwards run
    from the last read down), so the result is bitwise what the per-read tensors give (fused_dattn.py:343-346)."""
    cfg = chain_cfg(K, R, dtype)
    print(f"case acc chain K{K} R{R} {dtype}", flush=True)
    ha, ga = list_chain(cfg, accumulate=True)
    hp, gp = list_chain(cfg, accumulate=False)
    check_chain(ha, ga, cfg)
    assert torch.equal(ha, hp)
    for a, b in zip(grad_list(ga), grad_list(gp)):
        assert torch.equal(a, b)


def test_accumulating_list_reads_with_independent_bases():
    """FusedDattnReadAcc with bases that do not depend on the sources (each source's gradient then comes from the
    reads and its scale only): bitwise the per-read gradients, bf16, fp16 and fp32, three reads over four sources."""
    from loopback_amd import fused_dattn as FD
    d, b, t = 256, 1, 64
    gen = torch.Generator().manual_seed(21)
    for dtype in (torch.bfloat16, torch.float16, torch.float32):
        vals = [torch.randn(b, t, d, generator=gen).to(dtype) for _ in range(4)]
        bases = [torch.randn(b, t, d, generator=gen).to(dtype) for _ in range(4)]
        qs = torch.randn(3, d, generator=gen) * 0.5
        results = []
        for accumulate in (False, True):
            vs = [v.to(DEV).requires_grad_() for v in vals]
            acc = FD.DattnGradAccum()
            rs = [FD.rstd(v, 1e-6) for v in vs]
            loss = 0.0
            cbar = torch.ones(b, t, 1, device=DEV)
            prior = torch.ones(1, device=DEV)
            for s in range(1, 4):
                cb = torch.cat((cbar, torch.ones(b, t, 1, device=DEV)), -1)
                pr = torch.cat((prior, torch.ones(1, device=DEV)), -1)
                srcs = (*vs[:s + 1], *rs[:s + 1])
                base = bases[s].to(DEV)
                if accumulate:
                    out, tc = FD.FusedDattnReadAcc.apply(acc, s, qs[s - 1].to(DEV), base, cb, pr, *srcs)
                else:
                    out, tc = FD.FusedDattnRead.apply(qs[s - 1].to(DEV), base, cb, pr, *srcs)
                loss = loss + out.float().pow(2).mean()
                cbar, prior = tc, pr
            loss.backward()
            torch.cuda.synchronize()
            results.append([v.grad.cpu() for v in vs])
        for a, b_ in zip(*results):
            assert torch.equal(a, b_), dtype


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode", ["scores", "stack"])
def test_chain_with_saturated_reads(dtype, mode):
    """Queries large enough to saturate every read's softmax (q ~ N(0, 20^2): logits in the tens), through the
    stacked write's matrix-core scores and the reads: no worse against the exact chain than the reference chain in
    the same dtype (+ 1e-6 in fp32, + 2e-3 in bf16, the reference test's own slack, + 2.5e-4 in fp16)."""
    from loopback_amd.chain import ChainConfig
    cfg = ChainConfig("sat-K3R3", 256, 3, 3, 1, 200, dtype, True, q_std=20.0)
    print(f"case saturated {dtype} {mode}", flush=True)
    h, g = hip_chain(cfg, mode)
    hr, gr = ref_chain(cfg, None)
    h64, g64 = ref_chain(cfg, torch.float64)
    slack = 1e-6 if dtype == torch.float32 else lowp(2e-3, dtype)
    assert torch.isfinite(h).all()
    assert err_norm(h, h64) <= 2 * err_norm(hr, h64) + slack
    for a, b, c in zip(grad_list(g), grad_list(gr), grad_list(g64)):
        assert torch.isfinite(a).all()
        assert err_norm(a, c) <= 2 * err_norm(b, c) + slack


@pytest.mark.parametrize("K,R", [(2, 4), (3, 3)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("glue", ["1", "0"])
def test_layouts_agree(monkeypatch, K, R, dtype, glue):
    """The reference's layout contract (tests/test_dattn_stack.py:96-117, modeling_looped_transformer.py:137-139):
    the stacked layout without stored scores ('stack') and the list layout give the same forward bitwise, fp32,
    bf16 and fp16, in training and in evaluation -- the write stores each update's scale in the scale kernel's summation
    order and both run the same read kernel. Gradients: fp32 to 1e-6 norm-relative (the split backward sums in
    another order, as the reference's, whose bar this is). bf16: the stacked gradient of each update is one fp32
    sum rounded once, where the list layout rounds each read's term and autograd adds them in bf16 -- a deliberate
    difference; it stays within 1e-2 norm-relative of the list's and is no further from the exact (fp64) chain
    than the list's gradients are (+ 1e-3); fp16 likewise, to the bf16 bars 8 times tighter. The stored-score read
    ('scores') agrees with the list to 1e-5 (fp32) / 3e-2 (bf16; fp16 3.75e-3) norm-relative, the reference's bar
    (its scores come from the write, not the read)."""
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", glue)
    cfg = chain_cfg(K, R, dtype)
    print(f"case layouts K{K} R{R} {dtype} glue={glue}", flush=True)
    hl, gl = hip_chain(cfg, "list")
    hs, gs = hip_chain(cfg, "stack")
    hw, gw = hip_chain(cfg, "scores")
    assert torch.equal(hs, hl)
    if dtype == torch.float32:
        assert max(err_norm(a, b) for a, b in zip(grad_list(gs), grad_list(gl))) <= 1e-6
    else:
        _, g64 = ref_chain(cfg, torch.float64)
        for a, b, c in zip(grad_list(gs), grad_list(gl), grad_list(g64)):
            assert err_norm(a, b) <= lowp(1e-2, dtype)
            assert err_norm(a, c) <= err_norm(b, c) + lowp(1e-3, dtype)
    tol = 1e-5 if dtype == torch.float32 else lowp(3e-2, dtype)
    assert err_norm(hw, hl) <= tol
    assert max(err_norm(a, b) for a, b in zip(grad_list(gw), grad_list(gl))) <= tol
    ev = chain_cfg(K, R, dtype, backward=False)
    hl, _ = hip_chain(ev, "list", grad=False)
    hs, _ = hip_chain(ev, "stack", grad=False)
    assert torch.equal(hs, hl)


@pytest.mark.parametrize("K,R", [(3, 3), (1, 5)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode", ["stack", "scores"])
def test_fused_glue_matches_torch_glue(monkeypatch, K, R, dtype, mode):
    """The stacked read with the caller's glue in its kernels (FusedCombineStk) against the same read with the glue
    as torch ops (LOOP_DATTN_FUSE_GLUE=0): the forward is the same sequence of roundings, so the same bits; the
    gradients agree to round-off (autograd adds a proposal's gradient terms in another order). K = 1 makes every
    read an iteration end."""
    cfg = chain_cfg(K, R, dtype)
    print(f"case glue K{K} R{R} {dtype} {mode}", flush=True)
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", "0")
    ht, gt = hip_chain(cfg, mode)
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", "1")
    hf, gf = hip_chain(cfg, mode)
    assert torch.equal(hf, ht)
    tol = 1e-6 if dtype == torch.float32 else lowp(4e-3, dtype)
    worst = max(err_norm(a, b) for a, b in zip(grad_list(gf), grad_list(gt)))
    assert worst <= tol, worst


@pytest.mark.parametrize("K,R", [(3, 3), (1, 4)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("glue", ["1", "0"])
def test_proposal_gradient_through_update_kernel(monkeypatch, K, R, dtype, glue):
    """A read whose proposal (glue "1", FusedCombineStk) or base (glue "0", FusedDattnReadStk with the caller's torch
    glue; the base is the proposal at every read that is not an iteration end) is the write's h hands that gradient
    to the update-gradient kernel, which adds it as autograd would (round(round(dv) + g)); with the proposal a copy
    of h the same sum is formed by autograd. Every gradient agrees bitwise, and no handed-over gradient is left
    behind."""
    from loopback_amd.cell import LoopDeltaAttnRes
    from loopback_amd.chain import make_inputs
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", glue)
    cfg = chain_cfg(K, R, dtype)
    h0c, Dc, Q, G = make_inputs(cfg, "cpu")
    outs = []
    for copy in (False, True):
        cell = LoopDeltaAttnRes(cfg.d, cfg.R, cfg.K, beta=cfg.beta, eps=cfg.eps).to(DEV)
        with torch.no_grad():
            cell.query.copy_(Q.to(DEV))
        h0 = h0c.to(DEV).requires_grad_()
        D = [x.to(DEV).requires_grad_() for x in Dc]
        stack = cell.new_stack(h0.shape, h0.dtype, h0.device, mode="scores")
        h, deltas, keys, coeffs, prior = h0, [], [], None, None
        for s in range(cfg.N):
            l, blk = divmod(s, cfg.K)
            hs = h + D[s]
            deltas.append(stack.write(s, hs, h))
            h, coeffs, prior = cell.combine(hs.clone() if copy else hs, h0, deltas, coeffs, prior, l, blk,
                                            keys=keys, stack=stack)
        (h.float() * G.to(DEV)).sum().backward()
        torch.cuda.synchronize()
        assert not stack.gadd and not stack.neg
        outs.append([h0.grad.cpu(), cell.query.grad.cpu()] + [x.grad.cpu() for x in D])
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("case", ["other_eps", "copy"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode,glue", [("scores", "1"), ("scores", "0"), ("stack", "1"), ("stack", "0")])
def test_separate_scale_node_chain_matches_oracle(monkeypatch, case, dtype, mode, glue):
    """Scales the stack cannot take from the write go through the separate scale node (_RstdStk, the reference's
    DattnStack.rstd node, fused_dattn.py:698-722): "other_eps" asks stack.rstd for an eps other than the stack's
    (0.05 against 1e-6: the node recomputes R[s], and the reads' scores follow it), "copy" for the scale of a copy of
    the update (the node keeps the write's R[s]). Its backward assembles the update's gradient and hands (dv, -dv)
    and any proposal gradient a fused combine gave it to the write's backward (stack.neg). The chain, both glue
    settings (with glue in the kernels the proposal's gradient goes through that hand-off), both score modes,
    against the oracle chain whose keys use the scales' eps: the chain bars of test_chain_matches_oracle for the
    final state and every gradient (h0, every D_s, the query), and nothing handed over is left behind."""
    from loopback_amd import fused_dattn as FD
    from loopback_amd.chain import ChainConfig, make_cell, make_inputs
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", glue)
    key_eps = 0.05 if case == "other_eps" else 1e-6
    cfg = ChainConfig(f"rstdstk-{case}", 256, 2, 3, 1, 384, dtype, True, eps=key_eps, q_std=0.5)
    print(f"case separate scale node {case} {dtype} {mode} glue={glue}", flush=True)
    h0c, Dc, Qc, Gc = make_inputs(cfg, "cpu")
    h0 = h0c.to(DEV).requires_grad_()
    D = [x.to(DEV).requires_grad_() for x in Dc]
    cell = make_cell(cfg, Qc.to(DEV))
    stack = FD.DattnStack(cfg.N, h0.shape, dtype, DEV, query=cell.query if mode == "scores" else None, eps=1e-6)
    h, deltas, keys, coeffs, prior = h0, [], [], None, None
    for s in range(cfg.N):
        l, blk = divmod(s, cfg.K)
        x = h
        hs = x + D[s]
        deltas.append(stack.write(s, hs, x))
        keys.append(stack.rstd(s, deltas[-1].clone() if case == "copy" else deltas[-1], key_eps))
        assert type(keys[-1].grad_fn).__name__ == "_RstdStkBackward"
        h, coeffs, prior = cell.combine(hs, h0, deltas, coeffs, prior, l, blk, keys=keys, stack=stack)
    (h.float() * Gc.to(DEV)).sum().backward()
    torch.cuda.synchronize()
    assert not stack.gadd and not stack.neg
    check_chain(h.detach().cpu(), {"h0": h0.grad, "D": [x.grad for x in D], "query": cell.query.grad}, cfg)


def test_stack_and_list_read_bitwise_on_shared_scales():
    """One read, both layouts, the same sources and the same scale tensors: the same kernels give the same bits."""
    from loopback_amd import fused_dattn as FD
    n, b, t, d = 6, 2, 96, 768
    gen = torch.Generator().manual_seed(17)
    vals = [torch.randn(b, t, d, generator=gen).to(torch.bfloat16).to(DEV) for _ in range(n)]
    q = (torch.randn(d, generator=gen) * 0.3).to(DEV)
    base = torch.randn(b, t, d, generator=gen).to(torch.bfloat16).to(DEV)
    c0 = (torch.rand(n, generator=gen) + 0.1).to(DEV)
    cbar = (c0.view(1, 1, -1) + 0.1 * torch.randn(b, t, n, generator=gen).to(DEV)).contiguous()
    stack = FD.DattnStack(n, (b, t, d), torch.bfloat16, DEV)
    x = torch.zeros_like(vals[0])
    sv = [stack.write(s, vals[s], x) for s in range(n)]
    rs = [stack.rstd(s, sv[s], 1e-6) for s in range(n)]
    with torch.no_grad():
        o1, t1 = FD.FusedDattnReadStk.apply(stack, n - 1, q, base, cbar, c0, *sv, *rs)
        o2, t2 = FD.FusedDattnRead.apply(q, base, cbar, c0, *[v.clone() for v in sv], *[r.clone() for r in rs])
    assert torch.equal(o1, o2) and torch.equal(t1, t2)


def test_eval_chains():
    cfg = chain_cfg(3, 3, torch.bfloat16, backward=False)
    hl, _ = hip_chain(cfg, "list", grad=False)
    hs, _ = hip_chain(cfg, "stack", grad=False)
    hw, _ = hip_chain(cfg, "scores", grad=False)
    hr, _ = ref_chain(cfg, None, grad=False)
    for h in (hl, hs, hw):
        assert err_norm(h, hr) <= 1e-2


@pytest.mark.parametrize("policy", ["last", "zero"])
def test_eval_extra_iterations(policy):
    """Evaluation with more iterations than trained (scripts/eval_extra_visits.py): the queries remapped from a
    2-iteration cell drive a 4-iteration no-grad chain (no probability stores) that matches the oracle chain run
    with the same remapped queries."""
    from loopback_amd.cell import remap_query
    from loopback_amd.chain import make_inputs, run_chain
    cfg = chain_cfg(2, 4, torch.bfloat16, backward=False)
    h0, D, Q, G = make_inputs(cfg, "cpu")
    Qr = remap_query(Q[:2 * 2 - 1], 2, 2, 4, policy)
    for mode in ("scores", "stack", "list"):
        h, _, _ = run_chain(cfg, h0.to(DEV), [x.to(DEV) for x in D], Qr.to(DEV), G.to(DEV), mode, grad=False)
        torch.cuda.synchronize()
        states, _, _, _, _ = oracle_chain(cfg.K, cfg.R, h0, D, Qr, G, beta=cfg.beta, eps=cfg.eps, grad=False)
        assert err_norm(h.cpu(), states[-1]) <= 1e-2


@pytest.mark.parametrize("mode", ["stack", "scores"])
def test_kept_loss_holds_no_stack(mode):
    """After one chain's backward, keeping only its loss (and so its graph) keeps < 5 % of the stack's bytes
    (tests/test_dattn_stack.py:161-199)."""
    from loopback_amd.cell import LoopDeltaAttnRes
    K, R, N, d = 2, 4, 8192, 256

    def once():
        cell = LoopDeltaAttnRes(d, R, K, beta=0.75, eps=1e-6).to(DEV)
        with torch.no_grad():
            cell.query.normal_(0, 0.5)
        gen = torch.Generator().manual_seed(0)
        Ds = [(torch.randn(1, N, d, generator=gen) * 0.5).to(torch.bfloat16).to(DEV).requires_grad_()
              for _ in range(K * R)]
        h0 = (torch.randn(1, N, d, generator=gen) * 0.5).to(torch.bfloat16).to(DEV).requires_grad_()
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated()
        stack = cell.new_stack(h0.shape, h0.dtype, h0.device, mode=mode)
        h, deltas, keys, coeffs, prior = h0, [], [], None, None
        for s in range(K * R):
            l, blk = divmod(s, K)
            hs = h + Ds[s]
            deltas.append(stack.write(s, hs, h))
            h, coeffs, prior = cell.combine(hs, h0, deltas, coeffs, prior, l, blk, keys=keys, stack=stack)
        loss = (h.float() ** 2).mean()
        loss.backward()
        stack_bytes = 2 * (stack.V.numel() * stack.V.element_size() + stack.R.numel() * stack.R.element_size())
        del stack, h, hs, deltas, keys, coeffs, prior
        for p in (*Ds, h0, cell.query):
            p.grad = None
        torch.cuda.synchronize()
        return torch.cuda.memory_allocated() - before, stack_bytes, loss

    once()
    held, stack_bytes, kept = once()
    assert held < 0.05 * stack_bytes, (held, stack_bytes)
    del kept


@pytest.mark.parametrize("mode", ["list", "stack", "scores"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_empty_token_batch(mode, dtype):
    """A batch of no tokens ((1, 0, d)) through every layout, forward and backward: empty outputs and gradients of
    the right shapes, and a zero query gradient (a sum over no tokens); no kernel runs on an empty grid."""
    from loopback_amd.chain import ChainConfig, run_chain
    cfg = ChainConfig("empty-K2R2", 64, 2, 2, 1, 0, dtype, True)
    h0 = torch.zeros(1, 0, 64, dtype=dtype, device=DEV)
    D = [torch.zeros(1, 0, 64, dtype=dtype, device=DEV) for _ in range(cfg.N)]
    Q = torch.randn(cfg.N - 1, 64, device=DEV)
    G = torch.zeros(1, 0, 64, device=DEV)
    print(f"case empty {mode} {dtype}", flush=True)
    h, loss, grads = run_chain(cfg, h0, D, Q, G, mode)
    torch.cuda.synchronize()
    assert h.shape == (1, 0, 64) and loss.item() == 0.0
    assert grads["h0"].shape == (1, 0, 64) and all(g.shape == (1, 0, 64) for g in grads["D"])
    assert torch.equal(grads["query"], torch.zeros_like(Q))


@pytest.mark.parametrize("mode", ["list", "stack", "scores"])
def test_empty_token_batch_priors(mode):
    """With no tokens the read still hands back the next prior (the fused combine forms it in its kernel): every
    step's prior equals the oracle cell's."""
    from loopback_amd.cell import LoopDeltaAttnRes
    from oracle.reference_read import OracleCell
    K, R, d = 3, 2, 64
    Q = torch.randn(K * R - 1, d)
    cell = LoopDeltaAttnRes(d, R, K, beta=0.75, eps=1e-6).to(DEV)
    with torch.no_grad():
        cell.query.copy_(Q)
    ocell = OracleCell(d, R, K, 0.75, 1e-6, Q.double())
    h0 = torch.zeros(1, 0, d, device=DEV)
    stack = cell.new_stack(h0.shape, h0.dtype, h0.device, mode=mode)
    h, deltas, keys, coeffs, prior = h0, [], [], None, None
    oh, odeltas, okeys, ocoeffs, oprior = h0.cpu().double(), [], [], None, None
    with torch.no_grad():
        for s in range(K * R):
            l, blk = divmod(s, K)
            x, ox = h, oh
            hs, ohs = x + 0.0, ox + 0.0
            deltas.append(stack.write(s, hs, x) if stack is not None else hs - x)
            odeltas.append(ohs - ox)
            h, coeffs, prior = cell.combine(hs, h0, deltas, coeffs, prior, l, blk, keys=keys, stack=stack)
            oh, ocoeffs, oprior = ocell.combine(ohs, h0.cpu().double(), odeltas, ocoeffs, oprior, l, blk, keys=okeys)
            torch.cuda.synchronize()
            assert coeffs.shape == (1, 0, s + 1)
            assert torch.allclose(prior.cpu().double(), oprior, rtol=1e-6, atol=0), (s, prior, oprior)


def test_misuse_raises():
    """The reference module's RuntimeError cases (fused_dattn.py:371, 714, 733-734) and this build's limits, each
    raised before any launch: a stacked read whose base is not the stack's dtype or is not contiguous; a scale's
    backward before any read's; accumulating list reads run backward out of order (a source without a buffer); an
    rstd input of an unsupported dtype; a list read whose sources differ in dtype (the gate's refusal)."""
    from loopback_amd import fused_dattn as FD
    d, t, n = 64, 8, 2
    stack = FD.DattnStack(3, (1, t, d), torch.bfloat16, DEV)
    xs = [torch.randn(1, t, d, device=DEV, dtype=torch.bfloat16) for _ in range(3)]
    with torch.no_grad():
        ups = [stack.write(s, xs[s], torch.zeros_like(xs[s])) for s in range(n)]
        scales = [stack.rstd(s, ups[s], 1e-6) for s in range(n)]
    q = torch.zeros(d, device=DEV)
    cbar = torch.ones(1, t, n, device=DEV)
    c0 = torch.ones(n, device=DEV)
    with pytest.raises(RuntimeError, match="base"):
        FD.FusedDattnReadStk.apply(stack, 1, q, xs[2].float(), cbar, c0, *ups, *scales)
    wide = torch.randn(1, t, 2 * d, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="base"):
        FD.FusedDattnReadStk.apply(stack, 1, q, wide[..., :d], cbar, c0, *ups, *scales)

    lone = FD.DattnStack(2, (1, t, d), torch.float32, DEV)
    delta = torch.randn(1, t, d, device=DEV, requires_grad=True)
    r = lone.rstd(0, delta, 1e-6)
    with pytest.raises(RuntimeError, match="before any read"):
        r.sum().backward()

    vals = [torch.randn(1, t, d, device=DEV, requires_grad=True) for _ in range(3)]
    rs = [FD.rstd(v, 1e-6) for v in vals]
    acc = FD.DattnGradAccum()
    base = torch.randn(1, t, d, device=DEV)
    out1, _ = FD.FusedDattnReadAcc.apply(acc, 1, q, base, torch.ones(1, t, 2, device=DEV), torch.ones(2, device=DEV),
                                         *vals[:2], *rs[:2])
    out2, _ = FD.FusedDattnReadAcc.apply(acc, 2, q, base, torch.ones(1, t, 3, device=DEV), torch.ones(3, device=DEV),
                                         *vals, *rs)
    out1.sum().backward(retain_graph=True)      # read 1 first: only two buffers
    with pytest.raises(RuntimeError, match="out of order"):
        out2.sum().backward()

    with pytest.raises(RuntimeError, match="float64"):
        FD.rstd(torch.randn(1, t, d, device=DEV, dtype=torch.float64), 1e-6)
    mixed = [torch.randn(1, t, d, device=DEV), torch.randn(1, t, d, device=DEV, dtype=torch.bfloat16)]
    with pytest.raises(RuntimeError, match="unsupported"):
        FD.FusedDattnRead.apply(torch.zeros(d, device=DEV), torch.randn(1, t, d, device=DEV),
                                torch.ones(1, t, 2, device=DEV), torch.ones(2, device=DEV), *mixed,
                                *[FD.rstd(x, 1e-6) for x in mixed])


@pytest.mark.parametrize("mode", ["list", "stack", "scores"])
def test_chain_on_a_side_stream_is_bitwise_the_default_one(mode):
    """Every launch goes on the caller's current stream (the autograd thread's too, for the backward): a chain whose
    inputs are produced on a side stream right before it, run there fwd+bwd, gives the same bits as on the default
    stream (the kernels are deterministic; a launch on another stream could race those inputs)."""
    from loopback_amd.chain import ChainConfig, make_inputs, run_chain
    cfg = ChainConfig(f"side-{mode}", 256, 2, 3, 1, 2048, torch.bfloat16, True, q_std=0.5)
    h0, D, Q, G = make_inputs(cfg, "cpu")
    ref_h, ref_loss, ref_g = run_chain(cfg, h0.to(DEV), [x.to(DEV) for x in D], Q.to(DEV), G.to(DEV), mode)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        big = torch.randn(4096, 4096, device=DEV)
        for _ in range(4):
            big = big @ big.T * 1e-3             # keep the side stream busy ahead of the chain
        hd = (h0.to(DEV).float() + 0 * big[0, 0]).to(h0.dtype)   # the inputs depend on that work
        Dd = [x.to(DEV) for x in D]
        h, loss, g = run_chain(cfg, hd, Dd, Q.to(DEV), G.to(DEV), mode)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(h, ref_h) and torch.equal(loss, ref_loss)
    assert torch.equal(g["h0"], ref_g["h0"]) and torch.equal(g["query"], ref_g["query"])
    assert all(torch.equal(a, b) for a, b in zip(g["D"], ref_g["D"]))


@pytest.mark.parametrize("mode", ["list", "scores"])
@pytest.mark.parametrize("d", [512, 100])
def test_chains_from_two_threads_on_two_streams_at_once(mode, d):
    """The library keeps no state between calls (its entry points take every address and the stream, ctypes drops
    the GIL around each): two chains with different inputs, run fwd+bwd three times over from two host threads at
    once, each on a stream of its own, give the bits each gives alone on the default stream -- at a width of the
    row-layout kernels and one of the any-shape kernels (whose address tables are copied per call)."""
    import threading
    from loopback_amd.chain import ChainConfig, make_inputs, run_chain
    cfg = ChainConfig(f"threads-{mode}", d, 2, 3, 1, 4096, torch.bfloat16, True, q_std=0.5)
    h0, D, Q, G = make_inputs(cfg, "cpu")
    sets = [(h0, D, Q, G), (-h0, D[::-1], Q.flip(0), 2 * G)]
    sets = [(a.to(DEV), [x.to(DEV) for x in b], c.to(DEV), e.to(DEV)) for a, b, c, e in sets]
    refs = [run_chain(cfg, *s, mode) for s in sets]
    torch.cuda.synchronize()
    outs, errors = [None, None], []
    start = threading.Barrier(2)

    def work(k):
        try:
            stream = torch.cuda.Stream()
            stream.wait_stream(torch.cuda.default_stream())
            start.wait()
            with torch.cuda.stream(stream):
                for _ in range(3):
                    outs[k] = run_chain(cfg, *sets[k], mode)
            stream.synchronize()
        except Exception as exc:   # reported by the main thread
            errors.append(exc)

    print(f"case two threads {mode} d{d}", flush=True)
    threads = [threading.Thread(target=work, args=(k,)) for k in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a chain thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for (h, loss, g), (rh, rloss, rg) in zip(outs, refs):
        assert torch.equal(h, rh) and torch.equal(loss, rloss)
        assert torch.equal(g["h0"], rg["h0"]) and torch.equal(g["query"], rg["query"])
        assert all(torch.equal(a, b) for a, b in zip(g["D"], rg["D"]))


@pytest.mark.parametrize("K,R", [(2, 4), (3, 3), (1, 4)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [256, 100])
@pytest.mark.parametrize("glue", ["0", "1"])
def test_per_read_rounding_is_the_list_layout_bitwise(monkeypatch, K, R, dtype, d, glue):
    """LOOP_DATTN_GRAD_ROUNDING=per_read: the stacked layout (online scores; the caller's torch glue -- the reference
    trainer's own call sequence -- or the glue in the kernels) rounds each read's share of an update's gradient and
    adds the shares in the update dtype from the last read to the first, then the scale's term, as autograd adds the
    list layout's per-read gradients (and the iteration ends' shares of h0's gradient the same way): the final state
    and every gradient (h0, each update, the query) are the list layout's bit for bit, fp32, bf16 and fp16 -- the
    reference's contract (tests/test_dattn_stack.py:102-107), at a width of the row-layout kernels and one of the
    any-shape kernels (the default rounding is held to test_layouts_agree's bars)."""
    from loopback_amd.chain import ChainConfig
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", glue)
    cfg = ChainConfig(f"per-read-K{K}R{R}d{d}", d, K, R, 1, 160, dtype, True, q_std=0.5)
    print(f"case per-read rounding K{K} R{R} {dtype} d{d} glue={glue}", flush=True)
    hl, gl = hip_chain(cfg, "list")
    monkeypatch.setenv("LOOP_DATTN_GRAD_ROUNDING", "per_read")
    hs, gs = hip_chain(cfg, "stack")
    assert torch.equal(hs, hl)
    for name, a, b in zip(["h0", "query"] + [f"D{i}" for i in range(cfg.N)], grad_list(gs), grad_list(gl)):
        assert torch.equal(a.cpu(), b.cpu()), name


@pytest.mark.parametrize("mode", ["list", "stack", "scores"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_non_finite_input_stays_in_its_token(mode, dtype):
    """A NaN in one update at one token and an inf in another at a second token (the reference's reads propagate
    them through that token's scores and softmax): after the no-grad chain every other token's final state is
    bitwise the clean run's -- no tile, staging burst or score table carries one token's values into another's."""
    from loopback_amd.chain import ChainConfig, make_inputs, run_chain
    cfg = ChainConfig("nonfinite-K2R3", 256, 2, 3, 1, 300, dtype, False, q_std=0.5)
    h0, D, Q, G = make_inputs(cfg, "cpu")
    print(f"case non-finite {mode} {dtype}", flush=True)
    clean, _, _ = run_chain(cfg, h0.to(DEV), [x.to(DEV) for x in D], Q.to(DEV), G.to(DEV), mode, grad=False)
    Db = [x.clone() for x in D]
    Db[2][0, 17, 5] = float("nan")
    Db[4][0, 250, 100] = float("inf")
    dirty, _, _ = run_chain(cfg, h0.to(DEV), [x.to(DEV) for x in Db], Q.to(DEV), G.to(DEV), mode, grad=False)
    torch.cuda.synchronize()
    keep = torch.ones(cfg.n_tok, dtype=torch.bool)
    keep[[17, 250]] = False
    assert torch.equal(dirty[0, keep.to(DEV)], clean[0, keep.to(DEV)])
    assert not torch.isfinite(dirty[0, 17]).all() and not torch.isfinite(dirty[0, 250]).all()
