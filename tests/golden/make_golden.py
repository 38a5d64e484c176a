"""Writes the golden vectors of tests/golden/ with the oracle in fp64 (the reference ships none for this path):

  read_cases.npz   single reads at the list-layout interface (fp32 inputs): q, base, cbar, c0, the sources, upstream
                   gradients of out and tc -> out, tc and the closed-form gradients (oracle.analytic_backward) of q,
                   base, cbar and every source (through its value and its RMS scale)
  chain_case.npz   a K=2 x R=3 chain with blocks x -> x + D_s (fp32 inputs): the final state and the gradients of h0,
                   every D_s and the queries

    python tests/golden/make_golden.py        # rewrites both files (numpy .npz, no pickles)
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle.reference_read import analytic_backward, run_chain  # noqa: E402

READ_CASES = [(1, 8, 64, 2, 11), (2, 5, 64, 5, 12), (1, 16, 128, 8, 13), (1, 3, 256, 17, 14)]


def read_cases():
    out = {}
    for k, (b, t, d, n, seed) in enumerate(READ_CASES):
        g = torch.Generator().manual_seed(seed)
        vals = [torch.randn(b, t, d, generator=g) * (0.5 + 0.1 * i) for i in range(n)]
        base = torch.randn(b, t, d, generator=g)
        q = torch.randn(d, generator=g) * 0.3
        c0 = torch.rand(n, generator=g) * 0.9 + 0.1
        cbar = c0.view(1, 1, -1) + 0.2 * torch.randn(b, t, n, generator=g)
        up = torch.randn(b, t, d, generator=g)
        up2 = torch.randn(b, t, n, generator=g)
        ref = analytic_backward(q, base, cbar, c0, vals, up, up2, 1e-6)
        p = f"c{k}_"
        out[p + "shape"] = np.array([b, t, d, n])
        out[p + "values"] = np.stack([v.numpy() for v in vals])
        for name, x in (("base", base), ("q", q), ("c0", c0), ("cbar", cbar), ("up", up), ("up2", up2)):
            out[p + name] = x.numpy()
        for name in ("out", "tc", "dq", "dbase", "dcbar"):
            out[p + "ref_" + name] = np.asarray(ref[name])
        out[p + "ref_dv"] = np.stack(ref["dv"])
    out["n_cases"] = np.array(len(READ_CASES))
    return out


def chain_case():
    K, R, b, t, d = 2, 3, 1, 12, 64
    g = torch.Generator().manual_seed(21)
    h0 = torch.randn(b, t, d, generator=g)
    D = [torch.randn(b, t, d, generator=g) for _ in range(K * R)]
    Q = torch.randn(K * R - 1, d, generator=g) * 0.5
    G = torch.randn(b, t, d, generator=g)
    states, _, _, _, grads = run_chain(K, R, h0.double(), [x.double() for x in D], Q.double(), G.double())
    return {"K": np.array(K), "R": np.array(R), "h0": h0.numpy(), "D": np.stack([x.numpy() for x in D]),
            "Q": Q.numpy(), "G": G.numpy(), "ref_h": states[-1].numpy(), "ref_dh0": grads["h0"].numpy(),
            "ref_dD": np.stack([x.numpy() for x in grads["D"]]), "ref_dQ": grads["query"].numpy()}


if __name__ == "__main__":
    np.savez(os.path.join(HERE, "read_cases.npz"), **read_cases())
    np.savez(os.path.join(HERE, "chain_case.npz"), **chain_case())
    print("wrote", os.listdir(HERE))
