"""The oracle's read and gradients against what mathematics fixes, on CPU in fp64:
  * the key rms_no_affine, and the scale rstd_ref times its input, == torch.nn.functional.rms_norm without a weight
    (library routine);
  * autograd of read_core == the closed-form backward (analytic_backward, numpy, no autograd) for out, tc and the
    gradients of q, base, cbar and every source (through both its value and its RMS scale), with and without an
    upstream tc gradient;
  * torch.autograd.gradcheck (central differences) on a tiny read;
  * a pure-Python brute force of the paper's equation (c_{s,i} = B_s softmax_i(q . RMSNorm(d_i)/sqrt(d) + log c0))
    on a tiny chain against the oracle chain's states and tracked coefficients;
  * the zero-query identity out == base, tc == c0 bitwise in fp32 and bf16 (tests/test_fused_dattn.py:109-125).
A transposed operand, a missing r^3 term, a dropped Sacc or a wrong sign of dcbar fails one of these.
"""
import math

import numpy as np
import pytest
import torch

from oracle.reference_read import OracleCell, analytic_backward, paper_prior, read_core, rms_no_affine, run_chain


def make(b, t, d, n, dtype, seed, zero_query=False):
    g = torch.Generator().manual_seed(seed)
    values = [(torch.randn(b, t, d, generator=g) * (0.5 + 0.1 * i)).to(dtype) for i in range(n)]
    base = torch.randn(b, t, d, generator=g).to(dtype)
    q = torch.zeros(d) if zero_query else torch.randn(d, generator=g) * 0.3
    c0 = torch.rand(n, generator=g) * 0.9 + 0.1
    cbar = c0.view(1, 1, -1) + 0.2 * torch.randn(b, t, n, generator=g)
    up = torch.randn(b, t, d, generator=g)
    up2 = torch.randn(b, t, n, generator=g)
    return values, base, q, c0, cbar, up, up2


def test_key_is_rms_norm():
    x = torch.randn(3, 7, 96, dtype=torch.float64)
    ref = torch.nn.functional.rms_norm(x, (96,), weight=None, eps=1e-6)
    assert (rms_no_affine(x, 1e-6) - ref).abs().max().item() < 1e-14


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16])
def test_scale_is_rms_norm(dtype):
    """The scale alone (the oracle's rstd_ref and the module's own, fused_dattn.py:197-199): r x is torch's rms_norm
    of x, r being (..., 1). The module's is fp32 for every input (the reference's `delta.float()`); the oracle keeps
    fp64 for fp64 input (its exact evaluation) and scales bf16 input in fp32, as the reference does."""
    from loopback_amd import fused_dattn as FD
    from oracle.reference_read import rstd_ref
    x = (torch.randn(3, 7, 96, dtype=torch.float64) * 3.0).to(dtype)
    for fn, wide in ((rstd_ref, dtype == torch.float64), (FD.rstd_ref, False)):
        xf = x.double() if wide else x.float()
        ref = torch.nn.functional.rms_norm(xf, (96,), weight=None, eps=1e-6)
        r = fn(x, 1e-6)
        assert r.shape == (3, 7, 1) and r.dtype == xf.dtype
        tol = 1e-14 if wide else 2e-6
        assert ((r * xf) - ref).abs().max().item() <= tol * ref.abs().max().item()


@pytest.mark.parametrize("n", [1, 2, 5, 9])
@pytest.mark.parametrize("with_gt", [False, True])
def test_autograd_equals_closed_form(n, with_gt):
    values, base, q, c0, cbar, up, up2 = make(2, 5, 64, n, torch.float64, seed=11 * n + with_gt)
    values = [v.double().requires_grad_() for v in values]
    base = base.double().requires_grad_()
    q = q.double().requires_grad_()
    cbar = cbar.double().requires_grad_()
    c0 = c0.double()
    out, tc = read_core(q, base, cbar, c0, values, 1e-6)
    loss = (out * up.double()).sum() + ((tc * up2.double()).sum() if with_gt else 0.0)
    loss.backward()
    ref = analytic_backward(q, base, cbar, c0, values, up, up2 if with_gt else None, 1e-6)
    close = lambda a, b: np.abs(a.detach().numpy() - b).max() <= 1e-11 * max(1.0, np.abs(b).max())
    assert close(out, ref["out"]) and close(tc, ref["tc"])
    assert close(q.grad, ref["dq"]) and close(base.grad, ref["dbase"]) and close(cbar.grad, ref["dcbar"])
    for v, dv in zip(values, ref["dv"]):
        assert close(v.grad, dv)


def test_gradcheck_tiny_read():
    values, base, q, c0, cbar, _, _ = make(1, 2, 16, 3, torch.float64, seed=3)
    args = [q.double(), base.double(), cbar.double()] + [v.double() for v in values]
    args = [a.requires_grad_() for a in args]

    def fn(q_, base_, cbar_, *vals):
        out, tc = read_core(q_, base_, cbar_, c0.double(), list(vals), 1e-6)
        return out, tc
    assert torch.autograd.gradcheck(fn, args, eps=1e-6, atol=1e-8, rtol=1e-6)


def _brute_chain(K, R, h0, D, query, lam, eps):
    """Pure-Python loops over tokens / sources / features: the paper's equation, no incremental bookkeeping."""
    b, t, d = len(h0), len(h0[0]), len(h0[0][0])
    N = K * R
    states, coeffs = [], []
    h = h0
    deltas = []
    for s in range(N):
        hs = [[[h[bb][tt][k] + D[s][bb][tt][k] for k in range(d)] for tt in range(t)] for bb in range(b)]
        deltas.append([[[hs[bb][tt][k] - h[bb][tt][k] for k in range(d)] for tt in range(t)] for bb in range(b)])
        c0 = [lam ** ((s + 1) // K - i // K) for i in range(s + 1)]
        Bs = sum(c0)
        new_h, cs = [], []
        for bb in range(b):
            row_h, row_c = [], []
            for tt in range(t):
                logits = []
                for i in range(s + 1):
                    v = deltas[i][bb][tt]
                    rms = math.sqrt(sum(x * x for x in v) / d + eps)
                    z = sum((v[k] / rms) * (query[s - 1][k] if s >= 1 else 0.0) for k in range(d)) / math.sqrt(d)
                    logits.append(z + math.log(max(c0[i], 1e-8)))
                m = max(logits)
                e = [math.exp(x - m) for x in logits]
                c = [Bs * x / sum(e) for x in e]
                row_c.append(c)
                row_h.append([h0[bb][tt][k] + sum(c[i] * deltas[i][bb][tt][k] for i in range(s + 1))
                              for k in range(d)])
            new_h.append(row_h)
            cs.append(row_c)
        h = new_h
        states.append(h)
        coeffs.append(cs)
    return states, coeffs


def test_brute_force_paper_equation():
    K, R, lam, eps = 2, 2, 0.25, 1e-6
    g = torch.Generator().manual_seed(7)
    b, t, d = 1, 3, 8
    h0 = torch.randn(b, t, d, generator=g, dtype=torch.float64)
    D = [torch.randn(b, t, d, generator=g, dtype=torch.float64) for _ in range(K * R)]
    query = torch.randn(K * R - 1, d, generator=g, dtype=torch.float64) * 0.8
    G = torch.zeros(b, t, d, dtype=torch.float64)
    states, coeffs, _, _, _ = run_chain(K, R, h0, D, query, G, beta=1 - lam, eps=eps, grad=False)
    bs, bc = _brute_chain(K, R, h0.tolist(), [x.tolist() for x in D], query.tolist(), lam, eps)
    for s in range(K * R):
        assert (states[s] - torch.tensor(bs[s], dtype=torch.float64)).abs().max().item() < 1e-12, s
        assert (coeffs[s] - torch.tensor(bc[s], dtype=torch.float64)).abs().max().item() < 1e-12, s


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n", [2, 9, 16])
@pytest.mark.parametrize("boundary", [False, True])
def test_zero_query_identity_bitwise(dtype, n, boundary):
    b, t, d = 2, 8, 64
    values, proposal, _, prior, _, _, _ = make(b, t, d, n, dtype, seed=n, zero_query=True)
    h0 = torch.randn(b, t, d, generator=torch.Generator().manual_seed(99)).to(dtype)
    cell = OracleCell(d, 2, n if boundary else n + 1, 0.75, 1e-6, torch.zeros(2 * (n if boundary else n + 1) - 1, d))
    coeffs = prior[:-1].view(1, 1, -1).expand(b, t, -1).contiguous()
    out, tc, next_prior = cell.combine(proposal, h0, values, coeffs, prior[:-1], 0, n - 1)
    base = proposal + 0.75 * (h0 - proposal) if boundary else proposal
    assert torch.equal(out, base)
    assert torch.equal(tc, next_prior.view(1, 1, -1).expand(b, t, -1))


def test_prior_closed_form_values():
    # lam^(#iteration ends between write i and read s): K=3, s=4 -> floor(5/3)=1; i<3 -> lam^1, i>=3 -> lam^0
    p = paper_prior(3, 0.25, 4)
    assert p.tolist() == [0.25, 0.25, 0.25, 1.0, 1.0]
    p = paper_prior(3, 0.25, 5)          # the boundary read of iteration 1: floor(6/3) = 2
    assert p.tolist() == [0.0625, 0.0625, 0.0625, 0.25, 0.25, 0.25]
