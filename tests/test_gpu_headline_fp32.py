"""fp32 parity at the headline topology: the whole config-4 chain (d=2048, K=4, R=8 -> 32 updates and 31 reads,
T = 8 x 2048 = 16384 tokens, fwd+bwd) with fp32 updates, against the exact chain -- the oracle (the restated
reference read) in fp64 on the same inputs, run on the GPU beside the HIP chain because at this size it does not fit
the CPU's time. Every token and every gradient is compared: the final state, dL/dh0, every dL/dD_s and dL/dquery,
each within the fp32 bar of the target, max-abs error <= 1e-5 x RMS of the exact value. Both score modes (stored at
the write / formed by the read), both glue settings (the caller's torch glue around FusedDattnReadStk, as the
reference trainer calls it, and the glue in the kernels). At this size the reads run the 512-lane launch with 16-token
tiles (fp32 rows of 8 KiB) and every grid-capped kernel takes several tiles per workgroup.

The fp32 oracle chain (the literal reference read in fp32, also on the GPU) is measured beside it and printed, so a
failure shows whether the reference itself meets the bar on these inputs."""
import dataclasses

import pytest
import torch

from gpu_helpers import DEV
from oracle.reference_read import run_chain as oracle_chain

pytestmark = pytest.mark.gpu


def _names(N):
    return ["h", "h0", "query"] + [f"D{s}" for s in range(N)]


def _flat(h, grads):
    return [h, grads["h0"], grads["query"]] + list(grads["D"])


def _err(a, ref):
    """max |a - ref| / RMS(ref), on the device."""
    ref = ref.double()
    return ((a.double() - ref).abs().max() / ref.pow(2).mean().sqrt().clamp_min(1e-30)).item()


@pytest.fixture(scope="module")
def headline_fp32():
    from loopback_amd.chain import CONFIGS, make_inputs
    cfg = dataclasses.replace(CONFIGS["c4"], dtype=torch.float32, name="c4-d2048-N32-T16384-fp32-fwdbwd")
    assert (cfg.d, cfg.N, cfg.n_tok) == (2048, 32, 16384)
    print("case fp32 headline: the exact (fp64) oracle chain on the GPU", flush=True)
    h0, D, Q, G = make_inputs(cfg, DEV)
    states, _, _, _, ref = oracle_chain(cfg.K, cfg.R, h0.double(), [x.double() for x in D], Q.double(), G.double(),
                                        beta=cfg.beta, eps=cfg.eps, grad=True)
    exact = _flat(states[-1], ref)
    del states, ref
    print("case fp32 headline: the fp32 oracle chain on the GPU", flush=True)
    states, _, _, _, ref32 = oracle_chain(cfg.K, cfg.R, h0, D, Q, G, beta=cfg.beta, eps=cfg.eps, grad=True)
    e32 = [_err(a, b) for a, b in zip(_flat(states[-1], ref32), exact)]
    del states, ref32
    torch.cuda.empty_cache()
    worst = max(range(len(e32)), key=lambda i: e32[i])
    print(f"fp32 oracle chain vs exact: worst {e32[worst]:.3e} x RMS ({_names(cfg.N)[worst]}); h {e32[0]:.2e} "
          f"h0 {e32[1]:.2e} query {e32[2]:.2e} D max {max(e32[3:]):.2e}", flush=True)
    yield cfg, (h0, D, Q, G), exact
    del exact, h0, D, Q, G
    torch.cuda.empty_cache()


@pytest.mark.parametrize("mode,glue", [("scores", "1"), ("scores", "0"), ("stack", "1"), ("stack", "0")])
def test_headline_fp32_chain_against_exact(monkeypatch, headline_fp32, mode, glue):
    from loopback_amd.chain import run_chain
    monkeypatch.setenv("LOOP_DATTN_FUSE_GLUE", glue)
    cfg, (h0, D, Q, G), exact = headline_fp32
    print(f"case fp32 headline chain {mode} glue={glue}", flush=True)
    h, _, grads = run_chain(cfg, h0, D, Q, G, mode)
    torch.cuda.synchronize()
    errs = [_err(a, b) for a, b in zip(_flat(h, grads), exact)]
    names = _names(cfg.N)
    worst = max(range(len(errs)), key=lambda i: errs[i])
    print(f"HIP chain {mode} glue={glue} vs exact: worst {errs[worst]:.3e} x RMS ({names[worst]}); h {errs[0]:.2e} "
          f"h0 {errs[1]:.2e} query {errs[2]:.2e} D max {max(errs[3:]):.2e}", flush=True)
    assert all(torch.isfinite(x).all() for x in _flat(h, grads))
    assert errs[worst] <= 1e-5, {n: e for n, e in zip(names, errs) if e > 1e-5}
