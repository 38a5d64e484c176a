"""ORACLE -- test infrastructure only. A CPU restatement of the reference Loopback read, used as the checker of the
HIP path. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it; the product
(loopback_amd) never does.

What it restates (yancyou/Loopback, read as text, never imported):
  * `rms_no_affine`      looped_transformer.py:307-309  (the key of a stored update)
  * `rstd_ref`           fused_dattn.py:197-199         (the key's scale alone)
  * `paper_prior`        tests/loopback_audit/common.py:116-118 (c0_{s,i} = lam^(floor((s+1)/K) - floor(i/K)))
  * `OracleCell.combine` looped_transformer.py:371-424 (= modeling_looped_transformer.py:133-201 without the fused
                         branches): validation, the iteration-end blend, the coefficient bookkeeping and the
                         reference read itself -- fp32 scores from the normalized keys, the two softmaxes, the
                         installed coefficients, the correction cast to the activation dtype and summed source by
                         source in that dtype. Any torch dtype (fp32 for the literal reference, fp64 for truth).
  * `read_core`          the read alone, given base / cbar / c0 (what FusedDattnRead receives), same numerics.
  * `analytic_backward`  the closed-form backward of the read (fused_dattn.py:20-24) in numpy fp64, independent of
                         autograd; it pins the oracle's autograd gradients.
  * `run_chain`          the K x R chain with blocks x -> x + D_s (tests/loopback_audit/check_coefficients.py:25-40).

How each part is pinned (tests/test_oracle_*.py): closed forms C1/C2/C4/C5/C6 of the reference's audit (zero query
-> the paper prior and h0 coefficient 1; least-squares recovered coefficients == tracked ones; sum_i c_i = B_s;
boundary entry at lam; beta = 0 -> Plain Loop bitwise), the key against torch's own rms_norm, a pure-Python brute
force of the paper's equation on tiny inputs, and `analytic_backward` against autograd and central differences.
The reference ships no golden vectors for this path; tests/golden/ holds vectors this oracle wrote in fp64.
The code is device-agnostic torch: the checks run it on the CPU; one whole-model test runs the cell on the GPU beside
the HIP read, so that every other op of the model is the same kernel in both and the read alone can differ.
"""
from __future__ import annotations

import math

import numpy as np
import torch


def rms_no_affine(x: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm without a gain (looped_transformer.py:307-309)."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)


def rstd_ref(x: torch.Tensor, eps: float) -> torch.Tensor:
    """The scale alone, (..., 1) in fp32 or wider (fused_dattn.py:197-199)."""
    xf = x.float() if x.dtype in (torch.bfloat16, torch.float16) else x
    return torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)


def paper_prior(K: int, lam: float, s: int, dtype=torch.float64) -> torch.Tensor:
    """The decay prior of read s: c0_{s,i} = lam^(floor((s+1)/K) - floor(i/K)), i = 0..s (common.py:116-118)."""
    return torch.tensor([lam ** ((s + 1) // K - i // K) for i in range(s + 1)], dtype=dtype)


def _score_dtype(dtype: torch.dtype) -> torch.dtype:
    # the reference forms keys and scores with d.float(): fp32 for bf16 / fp32 activations; fp64 stays fp64 here
    return torch.float64 if dtype == torch.float64 else torch.float32


class OracleCell:
    """The reference read cell (looped_transformer.py:334-424) with its query given as a tensor (N-1, d)."""

    def __init__(self, dim: int, num_loops: int, num_blocks: int, beta: float, eps: float, query: torch.Tensor):
        if num_loops < 1 or num_blocks < 1:
            raise ValueError(f"delta_attnres needs positive num_loops/num_blocks, got {num_loops}/{num_blocks}")
        self.dim, self.num_loops, self.num_blocks = int(dim), int(num_loops), int(num_blocks)
        self.num_steps = self.num_loops * self.num_blocks
        self.beta, self.eps = float(beta), float(eps)
        if tuple(query.shape) != (self.num_steps - 1, self.dim):
            raise ValueError(f"query must be ({self.num_steps - 1}, {self.dim}), got {tuple(query.shape)}")
        self.query = query

    def combine(self, proposal, h0, deltas, coeffs, prior_coeffs, loop_idx, block_idx, keys=None):
        """looped_transformer.py:371-424, the reference read branch."""
        if not 0 <= block_idx < self.num_blocks:
            raise ValueError(f"delta_attnres block_idx={block_idx}, need [0,{self.num_blocks})")
        step = loop_idx * self.num_blocks + block_idx
        if step >= self.num_steps:
            raise ValueError(f"delta_attnres step {step} exceeds constructed depth {self.num_steps}")
        if len(deltas) != step + 1:
            raise ValueError(f"delta_attnres step {step} received {len(deltas)} deltas, expected {step + 1}")
        at_boundary = block_idx == self.num_blocks - 1
        base = proposal + self.beta * (h0 - proposal) if at_boundary else proposal
        cdt = _score_dtype(proposal.dtype)
        b, t, _ = proposal.shape
        one_tok = torch.ones(b, t, 1, dtype=torch.float32 if cdt == torch.float32 else cdt, device=proposal.device)
        one_prior = torch.ones(1, dtype=one_tok.dtype, device=proposal.device)
        base_coeffs = one_tok if coeffs is None else torch.cat((coeffs, one_tok), dim=-1)
        next_prior = one_prior if prior_coeffs is None else torch.cat((prior_coeffs, one_prior), dim=-1)
        if at_boundary:
            lam = 1.0 - self.beta
            base_coeffs = lam * base_coeffs
            next_prior = lam * next_prior
        if keys is not None and len(keys) < len(deltas):
            keys.append(rms_no_affine(deltas[-1].to(cdt), self.eps))
        if len(deltas) == 1:
            return base, base_coeffs, next_prior
        key_list = keys if keys is not None else [rms_no_affine(x.to(cdt), self.eps) for x in deltas]
        out, target = _read_from_keys(self.query[step - 1].to(cdt), base, base_coeffs, next_prior, deltas, key_list,
                                      self.dim)
        return out, target, next_prior


def _read_from_keys(q, base, cbar, c0, deltas, key_list, dim):
    """The body of the reference read (looped_transformer.py:410-424) from normalized keys."""
    inv = 1.0 / math.sqrt(dim)
    scores = torch.stack([torch.matmul(k, q) for k in key_list], dim=-1) * inv
    log_prior = torch.log(c0.clamp_min(1e-8))
    p0 = torch.softmax(log_prior, dim=-1)
    p = torch.softmax(scores + log_prior.view(1, 1, -1), dim=-1)
    mass = c0.sum()
    target = c0.view(1, 1, -1) + mass * (p - p0.view(1, 1, -1))
    coeff_delta = (target - cbar).to(base.dtype)
    correction = None
    for i, x in enumerate(deltas):
        term = coeff_delta[..., i].unsqueeze(-1) * x
        correction = term if correction is None else correction + term
    return base + correction, target


def read_core(q, base, cbar, c0, values, eps: float):
    """The read given what FusedDattnRead receives: query row q (d,), base, cbar (b, t, n), c0 (n,), the n values.
    Keys are the reference's (rms_no_affine of each value in the score dtype). Differentiable."""
    cdt = _score_dtype(base.dtype)
    keys = [rms_no_affine(v.to(cdt), eps) for v in values]
    return _read_from_keys(q.to(cdt), base, cbar, c0, values, keys, base.shape[-1])


def analytic_backward(q, base, cbar, c0, values, g, gt, eps: float):
    """Closed-form gradients of read_core in numpy fp64 (fused_dattn.py:20-24 plus the RMS-scale chain rule
    dr/dv = -r^3 v / d), written without autograd. Inputs are torch tensors (any dtype; computed in fp64).
    Returns dict(out, tc, dq, dbase, dcbar, dv: list) -- dv includes the path through the scale."""
    f = lambda t: t.detach().double().cpu().numpy()
    qn, c0n, cbn = f(q), f(c0), f(cbar)
    V = np.stack([f(v) for v in values], axis=-2)           # (b, t, n, d)
    gn, gtn = f(g), (np.zeros(cbn.shape) if gt is None else f(gt))
    d = V.shape[-1]
    inv = 1.0 / math.sqrt(d)
    r = 1.0 / np.sqrt((V * V).mean(-1) + eps)                # (b, t, n)
    z = r * (V @ qn) * inv
    lc = np.log(np.maximum(c0n, 1e-8))
    l = z + lc
    p = np.exp(l - l.max(-1, keepdims=True)); p /= p.sum(-1, keepdims=True)
    p0 = np.exp(lc - lc.max()); p0 /= p0.sum()
    M = c0n.sum()
    tc = c0n + M * (p - p0)
    w = tc - cbn
    out = f(base) + np.einsum("btn,btnd->btd", w, V)
    gd = np.einsum("btd,btnd->btn", gn, V)
    gp = M * (gd + gtn)
    sacc = (p * gp).sum(-1, keepdims=True)
    dz = p * (gp - sacc)
    dq = np.einsum("btn,btnd->d", dz * r, V) * inv
    dr = dz * z / r
    dv = w[..., None] * gn[..., None, :] + (dz * r * inv)[..., None] * qn
    dv = dv + (dr * (-r ** 3) / d)[..., None] * V          # through the scale r_i = rsqrt(mean v_i^2 + eps)
    return dict(out=out, tc=tc, dq=dq, dbase=gn, dcbar=-gd, dv=[dv[..., i, :] for i in range(V.shape[-2])])


def run_chain(K: int, R: int, h0, D, query, G, beta: float = 0.75, eps: float = 1e-6, grad: bool = True,
              use_keys: bool = True):
    """The K x R chain with blocks x -> x + D_s through OracleCell (the dtype of h0 / D is the activation dtype;
    query is used at its own dtype). Returns (states, coeffs, priors, loss, grads) where states[s] is the state
    after read s, grads = dict(h0, D, query) when grad."""
    N = K * R
    h0 = h0.detach().clone().requires_grad_(grad)
    D = [x.detach().clone().requires_grad_(grad) for x in D]
    query = query.detach().clone().requires_grad_(grad)
    cell = OracleCell(h0.shape[-1], R, K, beta, eps, query)
    states, coeffs_log, prior_log = [], [], []
    with torch.set_grad_enabled(grad):
        h, deltas, keys, coeffs, prior = h0, [], ([] if use_keys else None), None, None
        for s in range(N):
            l, blk = divmod(s, K)
            x = h
            hs = x + D[s]
            deltas.append(hs - x)
            h, coeffs, prior = cell.combine(hs, h0, deltas, coeffs, prior, l, blk, keys=keys)
            states.append(h)
            coeffs_log.append(coeffs)
            prior_log.append(prior)
        loss = (h.to(G.dtype) * G).sum()
        grads = None
        if grad:
            loss.backward()
            grads = {"h0": h0.grad, "D": [x.grad for x in D], "query": query.grad}
    return ([s.detach() for s in states], [c.detach() for c in coeffs_log], [p.detach() for p in prior_log],
            loss.detach(), grads)
