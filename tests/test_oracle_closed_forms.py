"""The oracle's chain against the closed forms of the reference's audit (tests/loopback_audit/check_coefficients.py:
91-145), fp64 on CPU. Blocks are x -> x + D_s with fixed D_s, so every state is h0 + sum_i c_i D_i exactly; the
coefficients are recovered per token by least squares and compared with:
  C1  zero queries: c_{s,i} = lam^(floor((s+1)/K) - floor(i/K)) at every read, h0 coefficient 1, last state closed form
  C2  the prior the cell carries == the paper's schedule at every read
  C4  learned queries: recovered == tracked coefficients, h0 coefficient 1, sum_i c_i == B_s, the query moves them
  C5  boundary reads: the newest update enters at lam (q = 0) / at its tracked target (q != 0)
  C6  beta = 0 and zero queries: bitwise the Plain Loop (h <- h + D_s)
A dropped decay, a wrong boundary index, a missing mass factor or a sign slip in the correction fails one of them.
"""
import pytest
import torch

from oracle.reference_read import paper_prior, run_chain

B, T, D_ = 2, 5, 64


def lstsq(x, h0, Ds):
    A = torch.stack([h0] + Ds, dim=-1)
    b, t, d, m = A.shape
    sol = torch.linalg.lstsq(A.reshape(b * t, d, m), x.reshape(b * t, d, 1)).solution.reshape(b, t, m)
    resid = (torch.einsum("btdm,btm->btd", A, sol) - x).abs().max().item()
    return sol[..., 0], sol[..., 1:], resid


def inputs(K, R):
    gen = torch.Generator().manual_seed(5 + K)
    Dl = [torch.randn(B, T, D_, generator=gen, dtype=torch.float64) * (0.5 + 0.1 * s) for s in range(K * R)]
    h0 = torch.randn(B, T, D_, generator=gen, dtype=torch.float64)
    query = torch.randn(K * R - 1, D_, generator=gen, dtype=torch.float64) * 0.6
    G = torch.randn(B, T, D_, generator=gen, dtype=torch.float64)
    return Dl, h0, query, G


TOPOS = [(4, 4), (3, 2)]


@pytest.mark.parametrize("K,R", TOPOS)
@pytest.mark.parametrize("lam", [0.25, 0.5])
def test_c1_c2_zero_query_is_the_paper_prior(K, R, lam):
    Dl, h0, query, G = inputs(K, R)
    states, coeffs, priors, _, _ = run_chain(K, R, h0, Dl, torch.zeros_like(query), G, beta=1 - lam, grad=False)
    for s in range(K * R):
        a, c, resid = lstsq(states[s], h0, Dl[: s + 1])
        want = paper_prior(K, lam, s)
        assert (c - want).abs().max().item() < 1e-9, s
        assert (a - 1).abs().max().item() < 1e-9
        assert resid < 1e-9
        assert (priors[s].double() - want).abs().max().item() < 1e-15            # C2
        assert (coeffs[s] - want).abs().max().item() < 1e-12                     # tracked == prior at q = 0
    last = states[-1] - (h0 + sum(lam ** (R - i // K) * Dl[i] for i in range(K * R)))
    assert last.abs().max().item() < 1e-9


@pytest.mark.parametrize("K,R", TOPOS)
@pytest.mark.parametrize("lam", [0.25, 0.5])
def test_c4_learned_query_tracked_coefficients(K, R, lam):
    Dl, h0, query, G = inputs(K, R)
    states, coeffs, priors, _, _ = run_chain(K, R, h0, Dl, query, G, beta=1 - lam, grad=False)
    moved = False
    for s in range(K * R):
        a, c, resid = lstsq(states[s], h0, Dl[: s + 1])
        assert (c - coeffs[s]).abs().max().item() < 1e-9, s
        assert (a - 1).abs().max().item() < 1e-9
        assert resid < 1e-9
        assert (coeffs[s].sum(-1) - priors[s].sum()).abs().max().item() < 1e-12   # mass B_s
        if s >= 1:
            moved |= (coeffs[s] - priors[s]).abs().max().item() > 1e-3
    assert moved


@pytest.mark.parametrize("K,R", TOPOS)
def test_c5_boundary_entry(K, R):
    lam = 0.25
    Dl, h0, query, G = inputs(K, R)
    s0, c0_, p0_, _, _ = run_chain(K, R, h0, Dl, torch.zeros_like(query), G, beta=1 - lam, grad=False)
    sq, cq, _, _, _ = run_chain(K, R, h0, Dl, query, G, beta=1 - lam, grad=False)
    for s in range(K - 1, K * R, K):
        _, c, _ = lstsq(sq[s], h0, Dl[: s + 1])
        assert (c[..., -1] - cq[s][..., -1]).abs().max().item() < 1e-9
        _, c0, _ = lstsq(s0[s], h0, Dl[: s + 1])
        assert (c0[..., -1] - lam).abs().max().item() < 1e-10


@pytest.mark.parametrize("K,R", TOPOS)
def test_c6_beta0_zero_query_is_plain_loop_bitwise(K, R):
    Dl, h0, query, G = inputs(K, R)
    states, _, _, _, _ = run_chain(K, R, h0, Dl, torch.zeros_like(query), G, beta=0.0, grad=False)
    h = h0
    for s in range(K * R):
        h = h + Dl[s]
        assert torch.equal(states[s], h), s
