"""Benchmark of the Loopback depth-attention read on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c4] [--mode scores] [--no-cpu-baseline]

A step is one pass of the read path over one batch: the K x R chain of the benchmark configuration (default
config 4: d=2048, K=4, R=8 -> N=32 updates, 31 reads, T = 8 x 2048 tokens, bf16 updates, fp32 scores), forward and
backward -- N writes (with the read-query scores), N-1 reads, their backwards, the updates' gradients -- with the
synthetic blocks x -> x + D_s and the caller's torch glue included. Inputs are resident in HBM before timing.

Prints ONE JSON line (rank 0): the headline metric (read tokens/s = T * steps / wall time), plus
  roofline      the dominant kernel (most time per pass): its compulsory bytes per launch / its mean launch
                duration, from HIP events on the launch stream during the last timed step, against 8 TB/s;
  chain         every library kernel of the pass: compulsory bytes / summed kernel time, and the reference
                dataflow's bytes (its backward read-modify-writes a gradient stack) over the same time and over
                the wall time;
  cpu_baseline  the CPU oracle (the restated reference read, fp32/bf16 torch on the host cores) on a bounded sample
                of the same chain (T reduced), fwd+bwd, tokens/s.
"""
from __future__ import annotations

import argparse
import contextlib
import gc
import json
import os
import statistics
import sys
import time

HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c4", choices=["c1", "c2", "c3", "c4"])
    ap.add_argument("--mode", default="scores", choices=["scores", "stack", "list"])
    ap.add_argument("--graph", action="store_true",
                    help="forward-only configs: time replays of the pass captured in a HIP graph (no host work)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-tokens", type=int, default=1024, help="tokens of the CPU baseline sample")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy 1 GiB device to device once (torch copy kernel): the known-size reference that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    return ap.parse_args()


def copy_calibration():
    import torch
    a = torch.empty(256 * 1024 * 1024, dtype=torch.float32, device="cuda")
    a.fill_(1.0)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": a.numel() * 4, "copy_calibration_bytes_written": b.numel() * 4}))


class KernelTimer:
    """HIP events around every library call, on the current (launch) stream; summed per kernel family."""

    def __init__(self):
        self.events = []

    @contextlib.contextmanager
    def __call__(self, name):
        import torch
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        yield
        b.record()
        self.events.append((name, a, b))

    def summary(self):
        import torch
        torch.cuda.synchronize()
        out = {}
        for name, a, b in self.events:
            ms = a.elapsed_time(b)
            t = out.setdefault(name, [0, 0.0])
            t[0] += 1
            t[1] += ms
        return {k: {"launches": v[0], "total_ms": v[1], "mean_us": 1e3 * v[1] / v[0]} for k, v in out.items()}


def family_bytes(cfg, mode):
    """Compulsory HBM bytes per pass (T tokens) of each kernel family of this build -- what each kernel must move:
    write 3 rows per token (h, x in; V out), read (n+2) (n sources, base in; out; with online scores the same, in one pass), backward pass 1
    (n+1) (n sources, g), update gradient (m+3) (the m output gradients of the reads holding the update, the update,
    the result and its negation for the write's x) -- in rows of e * d bytes; per-(token, source) fp32 scalars left
    out (< 1 %). With the caller's glue in the stacked read, a read at an iteration end also reads h0, the update
    gradient of each update a read took as its proposal adds the proposal's share (the add autograd would otherwise
    run) from that read's output gradient, which it reads anyway, and the iteration ends' shares of h0's gradient
    are summed once (blend_sum: one output gradient per iteration end in, one row out).
    Also the reference dataflow's total (its compulsory rows per token, e d (5N + 4 S2 + 4(N-1))), which moves more in
    its backward."""
    from loopback_amd.cell import fuse_glue
    from loopback_amd.chain import algorithmic_bytes_per_token
    e = 2 if cfg.dtype == torch_bf16() else 4
    N, T = cfg.N, cfg.n_tok
    S2 = N * (N + 1) // 2 - 1
    row = e * cfg.d * T
    fused = mode != "list" and fuse_glue()
    ends = sum(1 for s in range(1, N) if s % cfg.K == cfg.K - 1) if fused else 0
    read = "read_fwd" if mode == "scores" else "read_fwd_online"   # online scores: formed in the same pass
    fam = {"write_dots": 3 * N * row, read: (S2 + 2 * (N - 1) + ends) * row}
    if cfg.backward:
        fam["read_bwd1"] = (S2 + N - 1) * row
        fam["dv_assemble"] = ((N - 1) + N * (N - 1) // 2 + 3 * N) * row
        if ends:
            fam["blend_sum"] = (ends + 1) * row
    ref_total = algorithmic_bytes_per_token(N, cfg.d, e, backward=cfg.backward, dots=(mode == "scores"))["total"] * T
    return fam, ref_total


def torch_bf16():
    import torch
    return torch.bfloat16


def cpu_baseline(cfg, tokens):
    """The oracle chain on the host cores, fwd(+bwd), on `tokens` tokens of the same configuration."""
    import torch
    from oracle.reference_read import run_chain
    from loopback_amd.chain import make_inputs
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    h0, D, Q, G = make_inputs(cfg, "cpu", n_tok=tokens)
    run_chain(cfg.K, cfg.R, h0, D, Q, G, beta=cfg.beta, eps=cfg.eps, grad=cfg.backward)   # warm-up
    times, t_start = [], time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t_start < 10 and len(times) < 50):
        t0 = time.perf_counter()
        run_chain(cfg.K, cfg.R, h0, D, Q, G, beta=cfg.beta, eps=cfg.eps, grad=cfg.backward)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > 30:
            break
    med = statistics.median(times)
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), None)
    except OSError:
        pass
    return {"value": tokens / med, "unit": "read-tokens/s", "cores": torch.get_num_threads(), "cpu_model": model,
            "kind": "port",
            "sample": f"oracle chain (restated reference read, torch CPU) {cfg.name} with T={tokens} tokens, "
                      f"{'fwd+bwd' if cfg.backward else 'fwd'}, median of {len(times)} runs, {med:.3f} s/run"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the read shards by tokens "
              "across GPUs (only the query gradient is summed over them), but no multi-GPU figure is produced", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(3)
    if args.copy_calibration:
        copy_calibration()
        return
    from loopback_amd import fused_dattn as FD
    from loopback_amd.chain import CONFIGS, capture_forward, make_cell, make_inputs, run_chain

    cfg = CONFIGS[args.config]
    dev = torch.device("cuda", 0)
    h0, D, Q, G = make_inputs(cfg, dev)
    torch.cuda.synchronize()
    if args.graph:   # the forward pass as one HIP graph: no Python or launch work per pass
        if cfg.backward:
            print("bench.py: --graph times forward-only configurations (c2)", file=sys.stderr)
            sys.exit(2)
        graph, _ = capture_forward(cfg, h0, D, Q, args.mode)
        for _ in range(max(1, args.warmup)):
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            graph.replay()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        _, ref_bytes = family_bytes(cfg, args.mode)
        print(json.dumps({"metric": f"depth-read tokens/sec (fwd), {cfg.name}, HIP graph replay",
                          "value": cfg.n_tok * args.steps / elapsed, "unit": "read-tokens/s", "n_gpus": 1,
                          "steps": args.steps, "warmup": args.warmup, "ms_per_step": 1e3 * elapsed / args.steps,
                          "higher_is_better": True, "dtype": "bf16" if cfg.dtype == torch.bfloat16 else "fp32",
                          "formula_wall_gbs": ref_bytes * args.steps / elapsed / 1e9,
                          "config": {"workload": cfg.name, "mode": args.mode, "graph": True}}), flush=True)
        return

    cell = make_cell(cfg, Q)   # the model's read cell, made once (a training loop keeps its model)
    for _ in range(args.warmup):
        run_chain(cfg, h0, D, Q, G, args.mode, cell=cell)
    torch.cuda.synchronize()
    # The interpreter's long-lived objects (torch, the loaded modules) go to the permanent generation, as a serving
    # or training loop does after start-up: a full cyclic collection walks them all (~40 ms here) and would stall
    # the launch stream once every few steps; the steps themselves create no cycles that need collecting.
    gc.collect()
    gc.freeze()
    resident = torch.cuda.memory_allocated()   # the inputs and the cell, before any pass
    torch.cuda.reset_peak_memory_stats()
    timer = KernelTimer()
    t0 = time.perf_counter()
    for step in range(args.steps):
        if step == args.steps - 1:
            FD._TIMER = timer      # the last timed step: every library kernel bracketed by events on its stream
        run_chain(cfg, h0, D, Q, G, args.mode, cell=cell)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    FD._TIMER = None
    peak = torch.cuda.max_memory_allocated()
    ms_per_step = 1e3 * elapsed / args.steps
    ksum = timer.summary()
    fam, ref_bytes = family_bytes(cfg, args.mode)
    own_bytes = sum(fam.values())
    dom = max((k for k in fam if k in ksum), key=lambda k: ksum[k]["total_ms"])
    launches = ksum[dom]["launches"]
    bytes_per_launch = fam[dom] / launches
    mean_s = ksum[dom]["mean_us"] * 1e-6
    achieved = bytes_per_launch / mean_s / 1e9
    kernel_ms = sum(v["total_ms"] for v in ksum.values())
    # HBM bytes per launch of the dominant kernel from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary of
    # this configuration (profiles/traffic_chain_<config>.txt, copy-calibrated), when there is one for this mode
    traffic = None
    tr_path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"traffic_chain_{args.config}.txt")
    if os.path.exists(tr_path):
        with open(tr_path) as f:
            tr = json.load(f)
        if tr.get("mode") == args.mode:
            traffic = tr["hbm_bytes_per_launch"].get(dom)

    line = {
        "metric": ("depth-read tokens/sec (fwd+bwd), d=2048, N=32 stack" if args.config == "c4" else
                   f"depth-read tokens/sec ({'fwd+bwd' if cfg.backward else 'fwd'}), {cfg.name}"),
        "value": cfg.n_tok * args.steps / elapsed,
        "unit": "read-tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if cfg.dtype == torch.bfloat16 else "fp32",
        "data": "synthetic (seeded N(0,1) updates and h0, N(0,0.02^2) queries; blocks x -> x + D_s)",
        "config": {"workload": cfg.name, "d": cfg.d, "K": cfg.K, "R": cfg.R, "N": cfg.N, "tokens": cfg.n_tok,
                   "mode": args.mode, "backward": cfg.backward, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "algorithmic_bytes_per_launch": bytes_per_launch, "mean_launch_us": ksum[dom]["mean_us"],
                     "launches_per_step": launches},
        "chain": {"own_bytes_per_token": own_bytes / cfg.n_tok, "kernel_ms": kernel_ms,
                  "achieved_gbs": own_bytes / (kernel_ms * 1e-3) / 1e9,
                  "reference_formula_bytes_per_token": ref_bytes / cfg.n_tok,
                  "formula_gbs": ref_bytes / (kernel_ms * 1e-3) / 1e9,
                  "formula_wall_gbs": ref_bytes / (ms_per_step * 1e-3) / 1e9,
                  "kernels": {k: {"launches": v["launches"], "total_ms": round(v["total_ms"], 4),
                                  "gbs": (fam[k] / (v["total_ms"] * 1e-3) / 1e9) if k in fam else None}
                              for k, v in sorted(ksum.items())},
                  # device memory, as the reference's --bench reports it: the inputs resident before the passes,
                  # and the peak during them (the pass's stacks, saved tensors and gradients on top of the inputs)
                  "memory_gib": {"resident": resident / 2**30, "peak": peak / 2**30,
                                 "pass_peak": (peak - resident) / 2**30}},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(cfg, args.cpu_tokens)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
