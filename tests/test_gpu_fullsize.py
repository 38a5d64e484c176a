"""The benchmark configurations on the GPU. Config 1 (the reference's CPU case, 512 tokens) against the whole oracle
chain. Configs 2-4 at their full size (T = 16384 tokens), checked through properties that do not need the oracle to
run at that size, the stacked read both with the caller's glue as torch ops (the reference trainer's call sequence)
and inside the kernels:
  * the read is per token, so the HIP chain over all tokens restricted to a token subset must equal the oracle chain
    (the restated reference read in bf16, on the same inputs) over that subset -- final state, dL/dh0 and every
    dL/dD_s within 1e-2 norm-relative, and no further from the fp64 oracle than the reference read is;
  * the query gradient is a sum over tokens: HIP(all) == HIP(first half) + HIP(second half) to fp32 round-off, and
    HIP(subset) == oracle(subset);
  * config 2 runs both score modes (stored at the write / computed at the read): equal to bf16 rounding;
  * update tensors of more than 2^31 elements (4 GiB in bf16): per-token results at both ends of the range against
    the oracle on those tokens;
  * one stacked read at the headline shape (d=2048, 32 sources): zero query gives out == base and tc == c0 bitwise,
    and a learned query keeps the mass sum_i tc_i == B_s.
"""
import pytest
import torch

from gpu_helpers import DEV, err_norm, err_rms
from oracle.reference_read import run_chain as oracle_chain

pytestmark = pytest.mark.gpu

SUBSET = 48


def subset_idx(T):
    g = torch.Generator().manual_seed(123)
    idx = torch.randperm(T, generator=g)[:SUBSET].sort().values
    return torch.cat([torch.tensor([0, T - 1]), idx]).unique()


def flat(x):
    return x.reshape(-1, x.shape[-1])


@pytest.mark.parametrize("mode,glue", [("list", "1"), ("stack", "1"), ("scores", "1"), ("stack", "0"),
                                       ("scores", "0")])
def test_config1_forward_matches_oracle(monkeypatch, mode, glue):
    """Benchmark config 1, the reference's CPU case: d=768, K=2, R=4 (8 updates, 7 reads), 2 x 256 tokens, fp32,
    forward only; updates and h0 N(0,1), queries N(0, 0.02^2), lambda = 1/4. Through every read path, every state of
    the chain and every read's installed coefficients against the oracle chain: max-abs <= 1e-5 x RMS against the
    exact (fp64) chain and against the fp32 chain."""
    from loopback_amd.chain import CONFIGS, make_cell, make_inputs
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", glue)
    cfg = CONFIGS["c1"]
    assert (cfg.d, cfg.K, cfg.R, cfg.b, cfg.t, cfg.dtype, cfg.backward) == (768, 2, 4, 2, 256, torch.float32, False)
    print(f"case config1 {mode} glue={glue}", flush=True)
    h0, D, Q, G = make_inputs(cfg, "cpu")
    cell = make_cell(cfg, Q.to(DEV))
    states, coeffs_log = [], []
    with torch.no_grad():
        hd = h0.to(DEV)
        stack = cell.new_stack(hd.shape, hd.dtype, hd.device, mode=mode)
        h, deltas, keys, coeffs, prior = hd, [], [], None, None
        for s in range(cfg.N):
            l, blk = divmod(s, cfg.K)
            x = h
            hs = x + D[s].to(DEV)
            deltas.append(stack.write(s, hs, x) if stack is not None else hs - x)
            h, coeffs, prior = cell.combine(hs, hd, deltas, coeffs, prior, l, blk, keys=keys, stack=stack)
            states.append(h.cpu())
            coeffs_log.append(coeffs.cpu())
    torch.cuda.synchronize()
    for dt in (torch.float64, torch.float32):
        cast = (lambda x: x.to(dt))
        ref_states, ref_coeffs, _, _, _ = oracle_chain(cfg.K, cfg.R, cast(h0), [cast(x) for x in D], cast(Q),
                                                       cast(G), beta=cfg.beta, eps=cfg.eps, grad=False)
        e = [err_rms(a, b) for a, b in zip(states, ref_states)] + \
            [err_rms(a, b) for a, b in zip(coeffs_log[1:], ref_coeffs[1:])]
        assert max(e) <= 1e-5, (dt, e)


@pytest.mark.parametrize("key,glue", [("c2", "1"), ("c2", "0"), ("c3", "1"), ("c3", "0"), ("c4", "1"), ("c4", "0")])
def test_fullsize_chain_on_token_subset(monkeypatch, key, glue):
    from loopback_amd.chain import CONFIGS, make_inputs, run_chain
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", glue)
    cfg = CONFIGS[key]
    print(f"case fullsize {cfg.name} glue={glue}", flush=True)
    h0, D, Q, G = make_inputs(cfg, DEV)
    modes = ["scores", "stack"] if key == "c2" else ["scores"]
    outs = {}
    for mode in modes:
        h, _, grads = run_chain(cfg, h0, D, Q, G, mode)
        torch.cuda.synchronize()
        outs[mode] = (h, grads)
    idx = subset_idx(cfg.n_tok)
    sub = lambda x: flat(x)[idx.to(x.device)].unsqueeze(0).cpu()
    states, _, _, _, ref = oracle_chain(cfg.K, cfg.R, sub(h0), [sub(x) for x in D], Q.cpu(), sub(G), beta=cfg.beta,
                                        eps=cfg.eps, grad=cfg.backward)
    st64, _, _, _, ref64 = oracle_chain(cfg.K, cfg.R, sub(h0).double(), [sub(x).double() for x in D],
                                        Q.cpu().double(), sub(G).double(), beta=cfg.beta, eps=cfg.eps,
                                        grad=cfg.backward)
    h, grads = outs["scores"]

    def check(hip, r, r64):
        assert err_norm(hip, r) <= 1e-2
        assert err_norm(hip, r64) <= 2 * err_norm(r, r64) + 2e-3

    check(sub(h), states[-1], st64[-1])
    if key == "c2":
        assert err_norm(outs["stack"][0], h) <= 1e-2
    if cfg.backward:
        check(sub(grads["h0"]), ref["h0"], ref64["h0"])
        for a, b, c in zip(grads["D"], ref["D"], ref64["D"]):
            check(sub(a), b, c)
        # the query gradient: additivity over token halves, and the subset against the oracle
        T = cfg.n_tok
        half = T // 2
        parts = []
        for sl in (slice(0, half), slice(half, T)):
            cut = lambda x: flat(x)[sl].unsqueeze(0).contiguous()
            _, _, gp = run_chain(cfg, cut(h0), [cut(x) for x in D], Q, cut(G), "scores")
            parts.append(gp["query"])
        assert err_norm(parts[0] + parts[1], grads["query"]) <= 1e-4
        _, _, gs = run_chain(cfg, sub(h0).to(DEV), [sub(x).to(DEV) for x in D], Q, sub(G).to(DEV), "scores")
        check(gs["query"], ref["query"], ref64["query"])


@pytest.mark.parametrize("zero", [True, False])
def test_headline_read_identity_and_mass(zero):
    from loopback_amd import fused_dattn as FD
    N, b, t, d = 32, 8, 2048, 2048
    gen = torch.Generator(device=DEV).manual_seed(9)
    query = torch.zeros(N - 1, d, device=DEV) if zero else torch.randn(N - 1, d, device=DEV, generator=gen) * 0.05
    stack = FD.DattnStack(N, (b, t, d), torch.bfloat16, DEV, query=query, eps=1e-6)
    x = torch.zeros(b, t, d, device=DEV, dtype=torch.bfloat16)
    deltas = []
    for s in range(N):
        h = torch.randn(b, t, d, device=DEV, generator=gen).to(torch.bfloat16)
        deltas.append(stack.write(s, h, x))
    rs = [stack.rstd(s, deltas[s], 1e-6) for s in range(N)]
    lam = 0.25
    prior = torch.tensor([lam ** ((N) // 4 - i // 4) for i in range(N)], device=DEV)   # read N-1 (a boundary)
    cbar = prior.view(1, 1, -1).expand(b, t, -1).contiguous()
    base = torch.randn(b, t, d, device=DEV, generator=gen).to(torch.bfloat16)
    with torch.no_grad():
        out, tc = FD.FusedDattnReadStk.apply(stack, N - 1, query[N - 2], base, cbar, prior, *deltas, *rs)
    torch.cuda.synchronize()
    if zero:
        assert torch.equal(out, base)
        assert torch.equal(tc, cbar)
    else:
        mass = tc.double().sum(-1)
        assert (mass - prior.double().sum()).abs().max().item() <= 1e-5 * prior.sum().item()
        assert (tc - cbar).abs().max().item() > 1e-4         # the query moved the coefficients


@pytest.mark.parametrize("mode,glue,d", [("scores", "1", 2048), ("stack", "0", 2048), ("list", "1", 2048),
                                         ("scores", "1", 2050)])
def test_rows_past_2_31_elements(monkeypatch, mode, glue, d):
    """Every update tensor of more than 2^31 elements (T = 2^20 + 8 tokens x d = 2048, 4 GiB in bf16): a K = 1, R = 3
    chain, fwd+bwd (every read an iteration end), in the stacked and list layouts, and at d = 2050 on the any-shape
    kernels. Offsets past 2^31 elements must be formed in 64 bits everywhere; the per-token results at both ends of
    the range -- the final state, dL/dh0 and every dL/dD_s -- against the oracle chain on those tokens (the bars of
    test_fullsize_chain_on_token_subset), and the query gradient finite."""
    from loopback_amd.chain import ChainConfig, make_inputs, run_chain
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", glue)
    T = (1 << 20) + 8
    assert T * d > (1 << 31)
    cfg = ChainConfig("rows-past-2^31", d, 1, 3, 1, T, torch.bfloat16, True, q_std=0.5)
    print(f"case past 2^31 elements {mode} glue={glue} d{d}", flush=True)
    h0, D, Q, G = make_inputs(cfg, DEV)
    h, _, grads = run_chain(cfg, h0, D, Q, G, mode)
    torch.cuda.synchronize()
    idx = torch.cat([torch.arange(0, 24), torch.arange(T - 40, T)])
    sub = lambda x: flat(x)[idx.to(x.device)].unsqueeze(0).cpu()
    states, _, _, _, ref = oracle_chain(cfg.K, cfg.R, sub(h0), [sub(x) for x in D], Q.cpu(), sub(G), beta=cfg.beta,
                                        eps=cfg.eps, grad=True)
    st64, _, _, _, ref64 = oracle_chain(cfg.K, cfg.R, sub(h0).double(), [sub(x).double() for x in D],
                                        Q.cpu().double(), sub(G).double(), beta=cfg.beta, eps=cfg.eps, grad=True)

    def check(hip, r, r64):
        assert err_norm(hip, r) <= 1e-2
        assert err_norm(hip, r64) <= 2 * err_norm(r, r64) + 2e-3

    check(sub(h), states[-1], st64[-1])
    check(sub(grads["h0"]), ref["h0"], ref64["h0"])
    for a, b, c in zip(grads["D"], ref["D"], ref64["D"]):
        check(sub(a), b, c)
    assert torch.isfinite(grads["query"]).all()
    del h, grads, h0, D, G
    torch.cuda.empty_cache()
