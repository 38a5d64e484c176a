"""Per-launch cost of the library's streaming kernels: time = fixed + rows x per-row, fitted over the number of
sources n from back-to-back launches timed with HIP events on the launch stream, at T tokens and width d; and the
cost a kernel pays for the stores of the kernel before it (the caches write them back while it runs).

    python -m loopback_amd.launch_costs [--tokens 16384] [--widths 1024 2048] [--out FILE.md]

Rows are update-shaped rows of T x d bf16 (the read forward: n sources, its base and its output; backward pass 1:
n sources and g; the update gradient: n output gradients, the update, and its two outputs; the write: h and x in,
the update out, scoring n queries). Needs a GPU.
"""
from __future__ import annotations

import argparse

import numpy as np
import torch

from . import _lib as L

NS = (1, 2, 4, 8, 12, 16, 24, 32)


def _time_us(fn, reps: int = 20, warm: int = 3) -> float:
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps * 1e3


class _Bufs:
    """Synthetic operands of one width: 32 sources with their scales and scores, a base, output gradients."""

    def __init__(self, T: int, d: int, n_max: int = 32):
        dev, bf = torch.device("cuda", 0), torch.bfloat16
        g = torch.Generator(device=dev).manual_seed(0)
        self.T, self.d = T, d
        self.V = torch.randn(n_max, T, d, device=dev, generator=g).to(bf)
        self.R = torch.rand(n_max, T, device=dev, generator=g) + 0.5
        self.base = torch.randn(T, d, device=dev, generator=g).to(bf)
        self.out = torch.empty_like(self.base)
        self.dots = torch.randn(n_max, T, device=dev, generator=g) * 0.1
        self.cbar = torch.rand(T, n_max, device=dev, generator=g)
        self.c0 = torch.rand(n_max, device=dev, generator=g) + 0.1
        self.tc = torch.empty(T, n_max, device=dev)
        self.prob = torch.softmax(torch.randn(T, n_max, device=dev, generator=g), -1)
        self.g = torch.randn(T, d, device=dev, generator=g).to(bf)
        self.gt = torch.randn(T, n_max, device=dev, generator=g)
        self.dcbar = torch.empty(T, n_max, device=dev)
        self.dR = torch.zeros(n_max, T, device=dev)
        self.WZ = torch.randn(n_max, T, 2, device=dev, generator=g)
        self.G = torch.randn(n_max, T, d, device=dev, generator=g).to(bf)
        self.Q = torch.randn(n_max, d, device=dev, generator=g) * 0.02
        self.dv, self.dvn = torch.empty_like(self.base), torch.empty_like(self.base)
        self.parts = L.bwd1_parts(T, d)
        self.dq = torch.empty(self.parts, d, device=dev)
        self.st = torch.cuda.current_stream().cuda_stream
        # the write: a table of 32 read queries and their bf16 parts (the matrix cores' operand), its outputs
        self.Qw = torch.randn(32, d, device=dev, generator=g) * 0.02
        self.qb = torch.empty(int(L.LIB.ldr_query_parts_elems(32, d)), dtype=bf, device=dev)
        L.check(L.LIB.ldr_split_queries(self.Qw.data_ptr(), 32, d, self.qb.data_ptr(), self.st), "split_queries")
        self.W = torch.empty_like(self.base)
        self.Rw = torch.empty(T, device=dev)
        self.dw = torch.empty(32, T, device=dev)

    def launcher(self, kind: str, n: int):
        """(fn, rows) for one launch of `kind` over n sources."""
        lib, T, d, st = L.LIB, self.T, self.d, self.st
        vp = L.u64_array([self.V[i].data_ptr() for i in range(n)])
        rp = L.u64_array([self.R[i].data_ptr() for i in range(n)])

        def check(code):
            if code:
                L.check(code, kind)
        if kind == "read_fwd":
            return (lambda: check(lib.ldr_read_fwd(
                vp, rp, n, self.dots.data_ptr(), T, self.base.data_ptr(), None, 0.0, self.cbar.data_ptr(), n,
                self.c0.data_ptr(), n, 1.0, d ** -0.5, self.out.data_ptr(), self.tc.data_ptr(), self.prob.data_ptr(),
                None, T, d, L.BF16, st))), n + 2
        if kind == "read_bwd1":
            drp = L.u64_array([self.dR[i].data_ptr() for i in range(n)])
            return (lambda: check(lib.ldr_read_bwd1(
                vp, rp, n, self.g.data_ptr(), self.gt.data_ptr(), self.prob.data_ptr(), self.dots.data_ptr(), T,
                self.tc.data_ptr(), self.cbar.data_ptr(), n, self.c0.data_ptr(), n, 1.0, d ** -0.5,
                self.dcbar.data_ptr(), n, drp, 1, self.WZ.data_ptr(), T, self.dq.data_ptr(), d, None, None, 0.0, T, d,
                L.BF16, st))), n + 1
        if kind == "write":   # n: the queries scored, the last n of the table's 32; h = V[0], x = V[1]
            return (lambda: check(lib.ldr_write_dots(
                self.V[0].data_ptr(), self.V[1].data_ptr(), self.W.data_ptr(), self.Rw.data_ptr(), self.Qw.data_ptr(),
                self.qb.data_ptr(), 32, 32 - n, self.dw.data_ptr(), T, d, T, 1e-6, L.BF16, st))), 3
        if kind == "dv_assemble":
            gp = L.u64_array([self.G[i].data_ptr() for i in range(n)])
            wp = L.u64_array([self.WZ[i].data_ptr() for i in range(n)])
            qp = L.u64_array([self.Q[i].data_ptr() for i in range(n)])
            return (lambda: check(lib.ldr_dv_assemble(
                gp, wp, qp, n, self.V[0].data_ptr(), self.R[0].data_ptr(), self.R[1].data_ptr(),
                self.G[n - 1].data_ptr(), 0.0, 0, self.dv.data_ptr(), self.dvn.data_ptr(), T, d, L.BF16, st))), n + 3
        raise ValueError(kind)


def fit(bufs: _Bufs, kind: str) -> dict:
    xs, ys = [], []
    for n in NS:
        fn, rows = bufs.launcher(kind, n)
        xs.append(rows)
        ys.append(_time_us(fn))
    A = np.vstack([np.ones(len(xs)), xs]).T
    fixed, per_row = np.linalg.lstsq(A, np.array(ys), rcond=None)[0]
    row_bytes = bufs.T * bufs.d * 2
    return {"fixed_us": float(fixed), "per_row_us": float(per_row),
            "marginal_tbs": row_bytes / (per_row * 1e-6) / 1e12, "times_us": ys, "rows": xs}


def after_stores(bufs: _Bufs, kind: str = "read_fwd", n: int = 16, reps: int = 12) -> dict:
    """One launch of `kind` (n sources; for the write, n queries scored) timed alone (events just around it), after:
    an idle GPU, a read-only kernel (a sum over 64 MiB), and a torch add writing 64 MiB with ordinary stores."""
    fn, _ = bufs.launcher(kind, n)
    a, b = bufs.G[n], bufs.G[n + 1] if n + 1 < bufs.G.shape[0] else bufs.G[0]
    c = torch.empty_like(a)
    res = {}
    for name, before in (("idle GPU", None), ("read-only kernel", lambda: a.sum()),
                         ("64 MiB of stores", lambda: torch.add(a, b, out=c))):
        ts = []
        for _ in range(reps):
            torch.cuda.synchronize()
            if before is not None:
                before()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e3)
        ts = sorted(ts)[1:-1]
        res[name] = sum(ts) / len(ts)
    return res


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--tokens", type=int, default=16384)
    ap.add_argument("--widths", type=int, nargs="+", default=[1024, 2048])
    ap.add_argument("--out", default=None, help="write the markdown table here too")
    args = ap.parse_args()
    if not torch.cuda.is_available():
        raise SystemExit("launch_costs: needs a GPU")
    lines = [f"Per-launch cost, T = {args.tokens}, bf16 (back-to-back launches, HIP events; fit over n in {NS})", "",
             "| width | kernel | fixed us | us per row | marginal TB/s | times us (by n) |", "|---|---|---|---|---|---|"]
    stores = None
    for d in args.widths:
        bufs = _Bufs(args.tokens, d)
        for kind in ("read_fwd", "read_bwd1", "dv_assemble"):
            r = fit(bufs, kind)
            lines.append(f"| {d} | {kind} | {r['fixed_us']:.1f} | {r['per_row_us']:.2f} | {r['marginal_tbs']:.2f} | "
                         + ", ".join(f"{t:.1f}" for t in r["times_us"]) + " |")
            print(lines[-1], flush=True)
        wt = {nq: _time_us(bufs.launcher("write", nq)[0]) for nq in (0, 1, 16, 17, 32)}
        lines.append(f"| {d} | write (3 rows; by queries scored 0, 1, 16, 17, 32) | - | - | "
                     f"{3 * bufs.T * d * 2 / (wt[0] * 1e-6) / 1e12:.2f} (no scores) | "
                     + ", ".join(f"{t:.1f}" for t in wt.values()) + " |")
        print(lines[-1], flush=True)
        if d == max(args.widths):
            stores = {kind: after_stores(bufs, kind) for kind in ("read_fwd", "write")}
        del bufs
        torch.cuda.empty_cache()
    lines += ["", f"One launch (d = {max(args.widths)}; the read forward over 16 sources, the write scoring 16 queries) "
              "timed alone after:", "", "| before | read_fwd us | write us |", "|---|---|---|"]
    lines += [f"| {k} | {stores['read_fwd'][k]:.1f} | {stores['write'][k]:.1f} |" for k in stores["read_fwd"]]
    print("\n".join(lines[-6:]), flush=True)
    if args.out:
        with open(args.out, "w") as f:
            f.write("\n".join(lines) + "\n")


if __name__ == "__main__":
    main()
