"""The synthetic K x R chain that exercises the read the way the model's layer loop does.

Blocks are replaced by fixed maps x -> x + D_s (the reference's audit harness, tests/loopback_audit/
check_coefficients.py:25-40; the stacked-layout test's chain, tests/test_dattn_stack.py:68-92), so every state is
h0 + sum_i c_i d_i exactly and the read is the only real computation. Per step s = l K + blk:

    x = h;  hs = x + D_s;  d_s = stack.write(s, hs, x)  (or hs - x);  h, coeffs, prior = cell.combine(hs, h0, ...)

and the loss is sum(h.float() * G). The layer-loop shape follows modeling_looped_transformer.py:446-481.

The benchmark configurations (`CONFIGS`): tokens are b x t = 8 x 2048 unless stated; updates N(0,1), h0
N(0,1), queries N(0, 0.02^2), lambda = 1/4, eps = 1e-6, seeds 0 (h0), 1 (D), 2 (queries), 3 (G).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .cell import LoopDeltaAttnRes


@dataclass(frozen=True)
class ChainConfig:
    name: str
    d: int
    K: int
    R: int
    b: int
    t: int
    dtype: torch.dtype
    backward: bool
    beta: float = 0.75
    eps: float = 1e-6
    q_std: float = 0.02

    @property
    def N(self) -> int:
        return self.K * self.R

    @property
    def n_tok(self) -> int:
        return self.b * self.t


CONFIGS = {
    "c1": ChainConfig("c1-cpu-ref-d768-N8-T512-fp32-fwd", 768, 2, 4, 2, 256, torch.float32, False),
    "c2": ChainConfig("c2-d768-N8-T16384-bf16-fwd", 768, 2, 4, 8, 2048, torch.bfloat16, False),
    "c3": ChainConfig("c3-d1024-N12-T16384-bf16-fwdbwd", 1024, 3, 4, 8, 2048, torch.bfloat16, True),
    "c4": ChainConfig("c4-d2048-N32-T16384-bf16-fwdbwd", 2048, 4, 8, 8, 2048, torch.bfloat16, True),
}


def algorithmic_bytes_per_token(N: int, d: int, elt: int, backward: bool = True, dots: bool = True) -> dict:
    """Compulsory HBM bytes per token of one chain through the read path (the stacked dataflow of the reference):
    writes 3N (h, x in; V out; the DOTS-off form adds an rstd pass, 4N), forward reads sum_s (n+2), backward pass 1
    sum_s (n+1), pass 2 sum_s 1 + N + 2(S2 - N) (dV written on the first backward, read-modify-written after), the
    scale gradient 3N, in units of elt * d bytes; S2 = N(N+1)/2 - 1 source visits. Scalars excluded."""
    S2 = N * (N + 1) // 2 - 1
    reads = N - 1
    unit = elt * d
    parts = {
        "write": (3 if dots else 4) * N * unit,
        "read_fwd": (S2 + 2 * reads) * unit,
    }
    if backward:
        parts["bwd1"] = (S2 + reads) * unit
        parts["bwd2"] = (reads + N + 2 * (S2 - N)) * unit
        parts["rstd_bwd"] = 3 * N * unit
    parts["total"] = sum(parts.values())
    return parts


def make_inputs(cfg: ChainConfig, device, n_tok: int | None = None, q_std: float | None = None):
    """h0, D (list of N), query (N-1, d) fp32, G (fp32) for the chain, drawn on `device` from generators seeded
    0 (h0), 1 (D), 2 (query), 3 (G). A test that compares devices draws once and copies. n_tok overrides the
    token count (b = 1)."""
    T = cfg.n_tok if n_tok is None else n_tok
    shape = (1, T, cfg.d) if n_tok is not None else (cfg.b, cfg.t, cfg.d)
    dev = torch.device(device)
    gens = [torch.Generator(device=dev).manual_seed(k) for k in range(4)]
    h0 = torch.randn(shape, generator=gens[0], device=dev).to(cfg.dtype)
    D = [torch.randn(shape, generator=gens[1], device=dev).to(cfg.dtype) for _ in range(cfg.N)]
    std = cfg.q_std if q_std is None else q_std
    Q = torch.randn((cfg.N - 1, cfg.d), generator=gens[2], device=dev) * std
    G = torch.randn(shape, generator=gens[3], device=dev)
    return h0, D, Q, G


def chain_forward(cell, h0, D, K: int, mode: str):
    """The chain's forward through `cell` (blocks x -> x + D_s, the stacked write in the stacked modes)."""
    stack = cell.new_stack(h0.shape, h0.dtype, h0.device, mode=mode)
    h, deltas, keys, coeffs, prior = h0, [], [], None, None
    for s in range(len(D)):
        l, blk = divmod(s, K)
        x = h
        hs = x + D[s]
        deltas.append(stack.write(s, hs, x) if stack is not None else hs - x)
        h, coeffs, prior = cell.combine(hs, h0, deltas, coeffs, prior, l, blk, keys=keys, stack=stack)
    return h


def capture_forward(cfg: ChainConfig, h0, D, Q, mode: str):
    """A HIP graph of the no-grad chain forward on the static inputs h0, D (their contents may change between
    replays, not their storage). Returns (graph, out): graph.replay() recomputes out."""
    cell = LoopDeltaAttnRes(cfg.d, cfg.R, cfg.K, beta=cfg.beta, eps=cfg.eps).to(h0.device)
    with torch.no_grad():
        cell.query.copy_(Q)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            chain_forward(cell, h0, D, cfg.K, mode)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = chain_forward(cell, h0, D, cfg.K, mode)
    graph.cell = cell   # keeps the query alive with the graph
    return graph, out


def capture_training(cfg: ChainConfig, h0, D, Q, G, mode: str):
    """The whole training pass -- the chain's forward and its backward from the loss sum(h.float() * G) -- captured
    as ONE HIP graph: every library launch takes its addresses and sizes by value and allocates nothing, and torch's
    allocations (the stack, the saved tensors, the gradients) come from the graph's private pool, so a pass replays
    with one graph launch and no host work per kernel. The backward is seeded with that loss's gradient, G in the
    updates' dtype (what (h.float() * G).sum().backward() passes to h). Returns step() -> (h, loss, grads): one pass
    on the static inputs h0, D, G (their contents may change between passes, not their storage), the loss summed
    eagerly after the replay; grads = {'h0', 'D', 'query'} alias the graph's buffers until the next step (clone
    them to keep them)."""
    cell = make_cell(cfg, Q)
    h0s = h0.detach().requires_grad_()
    Ds = [x.detach().requires_grad_() for x in D]

    def body():
        h = chain_forward(cell, h0s, Ds, cfg.K, mode)
        h.backward(G.to(cfg.dtype))
        return h

    def clear():
        for t in (h0s, *Ds, cell.query):
            t.grad = None

    side = torch.cuda.Stream()   # warm-up on a side stream, as torch's capture expects
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            clear()
            body()
    torch.cuda.current_stream().wait_stream(side)
    clear()                      # the captured backward then writes fresh gradient buffers of the graph's pool
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        h = body()
    grads = {"h0": h0s.grad, "D": [x.grad for x in Ds], "query": cell.query.grad}

    def step():
        graph.replay()
        return h.detach(), (h.float() * G).sum(), grads

    step.graph, step.cell = graph, cell
    return step


def make_cell(cfg: ChainConfig, Q) -> LoopDeltaAttnRes:
    """The chain's read cell with its query set to Q (on Q's device)."""
    cell = LoopDeltaAttnRes(cfg.d, cfg.R, cfg.K, beta=cfg.beta, eps=cfg.eps).to(Q.device)
    with torch.no_grad():
        cell.query.copy_(Q)
    return cell


def run_chain(cfg: ChainConfig, h0, D, Q, G, mode: str, grad: bool | None = None, cell=None):
    """One pass of the chain through the HIP read in `mode` ('scores', 'stack' or 'list'). Returns
    (h_final, loss, grads) with grads = {'h0', 'D': [...], 'query'} when grad (default cfg.backward); without grad
    the pass is the forward alone (a forward-only configuration has no loss: loss and grads are None). `cell` (from
    make_cell) is reused across passes, as a training loop keeps its model: its query gradient is reset each pass;
    without one, a cell is made from Q."""
    grad = cfg.backward if grad is None else grad
    if cell is None:
        cell = make_cell(cfg, Q)
    else:
        cell.query.grad = None
    h0 = h0.detach().requires_grad_(grad)
    D = [x.detach().requires_grad_(grad) for x in D]
    with torch.set_grad_enabled(grad):
        h = chain_forward(cell, h0, D, cfg.K, mode)
        loss = grads = None
        if grad:
            loss = (h.float() * G).sum()
            loss.backward()
            grads = {"h0": h0.grad, "D": [x.grad for x in D], "query": cell.query.grad}
    return h.detach(), None if loss is None else loss.detach(), grads
