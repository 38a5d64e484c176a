"""The committed golden vectors (tests/golden/, written by the fp64 oracle; the reference ships none for this path):
the oracle reproduces them on the CPU (a guard against the oracle drifting), and the HIP read matches them on the GPU
within the fp32 tolerance (max-abs <= 1e-5 x RMS)."""
import os

import numpy as np
import pytest
import torch

from oracle.reference_read import read_core, run_chain

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def cases():
    z = np.load(os.path.join(HERE, "read_cases.npz"))
    for k in range(int(z["n_cases"])):
        yield {name[len(f"c{k}_"):]: z[name] for name in z.files if name.startswith(f"c{k}_")}


def err_rms(a, ref):
    a, ref = np.asarray(a, dtype=np.float64), np.asarray(ref, dtype=np.float64)
    return np.abs(a - ref).max() / max(np.sqrt((ref ** 2).mean()), 1e-30)


def test_oracle_reproduces_read_cases():
    for c in cases():
        t = {k: torch.from_numpy(v).double() for k, v in c.items() if k != "shape"}
        vals = [v.requires_grad_() for v in t["values"].unbind(0)]
        q, base, cbar = t["q"].requires_grad_(), t["base"].requires_grad_(), t["cbar"].requires_grad_()
        out, tc = read_core(q, base, cbar, t["c0"], vals, 1e-6)
        ((out * t["up"]).sum() + (tc * t["up2"]).sum()).backward()
        assert err_rms(out.detach(), c["ref_out"]) < 1e-12 and err_rms(tc.detach(), c["ref_tc"]) < 1e-12
        assert err_rms(q.grad, c["ref_dq"]) < 1e-10 and err_rms(cbar.grad, c["ref_dcbar"]) < 1e-10
        assert max(err_rms(v.grad, r) for v, r in zip(vals, c["ref_dv"])) < 1e-10


def test_oracle_reproduces_chain_case():
    z = np.load(os.path.join(HERE, "chain_case.npz"))
    K, R = int(z["K"]), int(z["R"])
    D = [torch.from_numpy(x).double() for x in z["D"]]
    states, _, _, _, g = run_chain(K, R, torch.from_numpy(z["h0"]).double(), D, torch.from_numpy(z["Q"]).double(),
                                   torch.from_numpy(z["G"]).double())
    assert err_rms(states[-1], z["ref_h"]) < 1e-12
    assert err_rms(g["query"], z["ref_dQ"]) < 1e-10 and err_rms(g["h0"], z["ref_dh0"]) < 1e-10


@pytest.mark.gpu
def test_hip_read_matches_golden():
    from loopback_amd import fused_dattn as FD
    dev = torch.device("cuda", 0)
    for c in cases():
        t = {k: torch.from_numpy(v).float().to(dev) for k, v in c.items() if k != "shape"}
        vals = [v.contiguous().requires_grad_() for v in t["values"].unbind(0)]
        q, base, cbar = t["q"].requires_grad_(), t["base"].requires_grad_(), t["cbar"].contiguous().requires_grad_()
        rstds = [FD.rstd(v, 1e-6) for v in vals]
        out, tc = FD.FusedDattnRead.apply(q, base, cbar, t["c0"], *vals, *rstds)
        ((out * t["up"]).sum() + (tc * t["up2"]).sum()).backward()
        torch.cuda.synchronize()
        assert err_rms(out.detach().cpu(), c["ref_out"]) <= 1e-5
        assert err_rms(tc.detach().cpu(), c["ref_tc"]) <= 1e-5
        assert err_rms(q.grad.cpu(), c["ref_dq"]) <= 1e-5
        assert err_rms(base.grad.cpu(), c["ref_dbase"]) <= 1e-5
        assert err_rms(cbar.grad.cpu(), c["ref_dcbar"]) <= 1e-5
        assert max(err_rms(v.grad.cpu(), r) for v, r in zip(vals, c["ref_dv"])) <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["scores", "stack", "list"])
def test_hip_chain_matches_golden(mode):
    from loopback_amd.chain import ChainConfig, run_chain as hip_chain
    z = np.load(os.path.join(HERE, "chain_case.npz"))
    K, R = int(z["K"]), int(z["R"])
    dev = torch.device("cuda", 0)
    cfg = ChainConfig("golden", z["h0"].shape[-1], K, R, 1, z["h0"].shape[1], torch.float32, True)
    h, _, g = hip_chain(cfg, torch.from_numpy(z["h0"]).to(dev), [torch.from_numpy(x).to(dev) for x in z["D"]],
                        torch.from_numpy(z["Q"]).to(dev), torch.from_numpy(z["G"]).to(dev), mode)
    torch.cuda.synchronize()
    assert err_rms(h.cpu(), z["ref_h"]) <= 1e-5
    assert err_rms(g["h0"].cpu(), z["ref_dh0"]) <= 1e-5
    assert err_rms(g["query"].cpu(), z["ref_dQ"]) <= 1e-5
    assert max(err_rms(a.cpu(), b) for a, b in zip(g["D"], z["ref_dD"])) <= 1e-5
