"""Benchmark of the Loopback depth-attention read on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c4] [--mode scores] [--no-cpu-baseline]
                    [--no-extra-configs] [--dtype bf16|fp16|fp32] [--glue 0|1]

A step is one pass of the read path over one batch: the K x R chain of the benchmark configuration (default
config 4: d=2048, K=4, R=8 -> N=32 updates, 31 reads, T = 8 x 2048 tokens, bf16 updates, fp32 scores), forward and
backward -- N writes (with the read-query scores), N-1 reads, their backwards, the updates' gradients -- with the
synthetic blocks x -> x + D_s and the caller's glue included. Inputs are resident in HBM before timing. --dtype
times the same configuration with other update dtypes (fp16: the trainer's fp16 mixed precision); the default run
is the configuration's own dtype. --glue 0 runs the stacked read as the reference trainer calls it after the import
swap (FusedDattnReadStk with the caller's glue as torch ops, LOOP_DATTN_FUSE_GLUE=0); the default, 1, is the read
cell's own path, with that glue inside the read's kernels (FusedCombineStk).

Prints ONE JSON line (rank 0): the headline metric (read tokens/s = T * steps / wall time), plus
  roofline      the dominant kernel (most time per pass): the reference dataflow's algorithmic bytes per launch for
                that kernel (per launch: a read moves n sources, its base and its output) / its mean
                launch duration, from HIP events on the launch stream during the last timed step, against 8 TB/s;
                the HBM bytes per launch measured by rocprofv3 FETCH_SIZE / WRITE_SIZE for this source (the committed
                profile, labelled with the kernel source it was measured on);
  chain         every library kernel of the pass: this build's compulsory bytes / summed kernel time, and the
                reference dataflow's bytes (its backward read-modify-writes a gradient stack) over the same time and
                over the wall time; counter_gbs: the HBM bytes the FETCH_SIZE / WRITE_SIZE counters measured per
                launch of each family (the committed profile, labelled with the kernel source it was measured on)
                times this pass's launches, over the same families' kernel time;
  configs       configs 2 and 3 timed the same way (wall time per pass), eager and replayed from HIP graphs;
                configs 4 and 3 through the drop-in path the reference trainer runs (FusedDattnReadStk with the
                caller's torch glue: c4_torch_glue, c3_torch_glue);
                config 5, the LM training step with the read, and the same model as Plain Loop (the read's cost)
                (--no-extra-configs skips them);
  cpu_baseline  the CPU oracle (the restated reference read, torch on the host cores) on a bounded sample of the
                same chain (T reduced), fwd+bwd, read-tokens/s and effective GB/s; beside it config 1 (the
                reference's CPU case: d=768, N=8, 512 tokens, fp32, forward).
"""
from __future__ import annotations

import argparse
import contextlib
import dataclasses
import gc
import hashlib
import json
import os
import statistics
import subprocess
import sys
import time

HBM_PEAK_GBS = 8000.0
ROOT = os.path.dirname(os.path.abspath(__file__))


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c4", choices=["c1", "c2", "c3", "c4"])
    ap.add_argument("--mode", default="scores", choices=["scores", "stack", "list"])
    ap.add_argument("--dtype", default=None, choices=sorted(DTYPE_NAMES),
                    help="the updates' dtype (default: the configuration's own)")
    ap.add_argument("--glue", default=None, choices=["0", "1"],
                    help="LOOP_DATTN_FUSE_GLUE for the timed chain: 0 the caller's glue as torch ops around "
                         "FusedDattnReadStk (the reference trainer's calls), 1 the glue in the read's kernels "
                         "(default: the environment's setting, else 1)")
    ap.add_argument("--graph", action="store_true",
                    help="time replays of the pass captured in a HIP graph (no host work per kernel): the forward, "
                         "or a training pass's forward and backward, as one graph")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra-configs", action="store_true", help="skip the c2 / c3 timings of the default run")
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


DTYPE_NAMES = {"bf16": "bfloat16", "fp16": "float16", "fp32": "float32"}


def dtype_name(dtype) -> str:
    """The bench line's name of a torch dtype ("bf16", "fp16", "fp32")."""
    return {v: k for k, v in DTYPE_NAMES.items()}[str(dtype).replace("torch.", "")]


def with_dtype(cfg, name: str | None):
    """The configuration with its updates in dtype `name` ("bf16", "fp16", "fp32"; None or its own: unchanged),
    its name saying so."""
    import torch
    own = dtype_name(cfg.dtype)
    if name is None or name == own:
        return cfg
    return dataclasses.replace(cfg, dtype=getattr(torch, DTYPE_NAMES[name]), name=cfg.name.replace(own, name))


def elt_bytes(dtype) -> int:
    import torch
    return torch.empty(0, dtype=dtype).element_size()


def _shape(cfg, mode):
    from loopback_amd.cell import fuse_glue
    e = elt_bytes(cfg.dtype)
    N, T = cfg.N, cfg.n_tok
    S2 = N * (N + 1) // 2 - 1
    fused = mode != "list" and fuse_glue()
    ends = sum(1 for s in range(1, N) if s % cfg.K == cfg.K - 1) if fused else 0
    return e, N, T, S2, ends, e * cfg.d * T


def family_bytes(cfg, mode):
    """Compulsory HBM bytes per pass (T tokens) of each kernel family of this build -- what each kernel must move:
    write 3 rows per token (h, x in; V out), read (n+2) (n sources, base in; out; with online scores the same, in
    one pass), backward pass 1 (n+1) (n sources, g), update gradient (m+3) (the m output gradients of the reads
    holding the update, the update, the result and its negation for the write's x) -- in rows of e * d bytes;
    per-(token, source) fp32 scalars left out (< 1 %). With the caller's glue in the stacked read, a read at an
    iteration end also reads h0, the update gradient of each update a read took as its proposal adds the proposal's
    share (the add autograd would otherwise run) from that read's output gradient, which it reads anyway, and the
    iteration ends' shares of h0's gradient are summed once (blend_sum: one output gradient per iteration end in,
    one row out).
    Also the reference dataflow's total (its compulsory rows per token, e d (5N + 4 S2 + 4(N-1))), which moves more in
    its backward."""
    from loopback_amd.chain import algorithmic_bytes_per_token
    e, N, T, S2, ends, row = _shape(cfg, mode)
    read = "read_fwd" if mode == "scores" else "read_fwd_online"   # online scores: formed in the same pass
    fam = {"write_dots": 3 * N * row, read: (S2 + 2 * (N - 1) + ends) * row}
    if cfg.backward:
        fam["read_bwd1"] = (S2 + N - 1) * row
        fam["dv_assemble"] = ((N - 1) + N * (N - 1) // 2 + 3 * N) * row
        if ends:
            fam["blend_sum"] = (ends + 1) * row
    ref_total = algorithmic_bytes_per_token(N, cfg.d, e, backward=cfg.backward, dots=(mode == "scores"))["total"] * T
    return fam, ref_total


def reference_bytes(cfg, mode):
    """The reference dataflow's algorithmic bytes per pass of the work each kernel family does (its rows per
    token, without this build's extras): the write 3N, the reads sum_s (n + 2) (n sources, base, out), backward
    pass 1 sum_s (n + 1); the update gradient does the reference's backward pass 2 and scale-gradient
    accumulation, (N - 1) + N + 2 (S2 - N) + 3N. The fused blend's h0 rows (reads at an iteration end) are
    counted apart (`extra_rows_per_pass`). blend_sum has no counterpart in the reference's kernels."""
    e, N, T, S2, ends, row = _shape(cfg, mode)
    read = "read_fwd" if mode == "scores" else "read_fwd_online"
    out = {"write_dots": 3 * N * row, read: (S2 + 2 * (N - 1)) * row}
    if cfg.backward:
        out["read_bwd1"] = (S2 + N - 1) * row
        out["dv_assemble"] = ((N - 1) + N + 2 * (S2 - N) + 3 * N) * row
    return out, {read: ends}


def source_sha256() -> str:
    with open(os.path.join(ROOT, "loopback_amd", "csrc", "loopback_read.hip"), "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


@contextlib.contextmanager
def env_set(name: str, value: str):
    """os.environ[name] = value inside the block (the read's mode switches are read at every call)."""
    old = os.environ.get(name)
    os.environ[name] = value
    try:
        yield
    finally:
        if old is None:
            os.environ.pop(name, None)
        else:
            os.environ[name] = old


def committed_traffic_table(config, mode):
    """The committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary of this configuration and read mode with the glue in
    the kernels (profiles/traffic_chain_<config>.txt, copy-calibrated): HBM bytes per launch of each kernel family,
    and a label naming the kernel source it was measured on and whether that is this build's source."""
    path = os.path.join(ROOT, "profiles", f"traffic_chain_{config}.txt")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        tr = json.load(f)
    if tr.get("mode") != mode or str(tr.get("glue", "1")) != "1":
        return None, None
    measured_on = tr.get("source_sha256")
    label = {"file": os.path.relpath(path, ROOT), "measured_on_source_sha256": measured_on,
             "measured_at_commit": tr.get("commit"), "this_source_sha256": source_sha256(),
             "current": measured_on == source_sha256()}
    return tr.get("hbm_bytes_per_launch", {}), label


def committed_traffic(config, mode, dom):
    """HBM bytes per launch of `dom` from committed_traffic_table, with its label."""
    table, label = committed_traffic_table(config, mode)
    if table is None or dom not in table:
        return None, None
    return table[dom], label


def counter_chain(table, ksum):
    """The chain's HBM GB/s from the counters: per family, the measured bytes per launch times this pass's launches,
    summed over the families the table holds, over those families' kernel time in this pass."""
    fams = [k for k in table if k in ksum]
    if not fams:
        return None
    measured = sum(table[k] * ksum[k]["launches"] for k in fams)
    ms = sum(ksum[k]["total_ms"] for k in fams)
    return {"counter_gbs": measured / (ms * 1e-3) / 1e9, "counter_bytes_per_pass": measured,
            "counter_kernel_ms": ms, "families": sorted(fams)}


def time_chain(cfg, mode, steps, warmup, timer=None):
    """Warm-up, then `steps` timed chain passes bracketed by synchronizations; returns (elapsed s, resident bytes,
    peak bytes). With `timer`, the last timed pass brackets every library kernel with events."""
    import torch
    from loopback_amd import fused_dattn as FD
    from loopback_amd.chain import make_cell, make_inputs, run_chain
    dev = torch.device("cuda", 0)
    h0, D, Q, G = make_inputs(cfg, dev)
    cell = make_cell(cfg, Q)   # the model's read cell, made once (a training loop keeps its model)
    for _ in range(warmup):
        run_chain(cfg, h0, D, Q, G, mode, cell=cell)
    torch.cuda.synchronize()
    # The interpreter's long-lived objects (torch, the loaded modules) go to the permanent generation, as a serving
    # or training loop does after start-up: a full cyclic collection walks them all (~40 ms here) and would stall
    # the launch stream once every few steps; the steps themselves create no cycles that need collecting.
    gc.collect()
    gc.freeze()
    resident = torch.cuda.memory_allocated()   # the inputs and the cell, before any pass
    torch.cuda.reset_peak_memory_stats()
    t0 = time.perf_counter()
    for step in range(steps):
        if timer is not None and step == steps - 1:
            FD._TIMER = timer      # the last timed step: every library kernel bracketed by events on its stream
        run_chain(cfg, h0, D, Q, G, mode, cell=cell)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    FD._TIMER = None
    gc.unfreeze()
    peak = torch.cuda.max_memory_allocated()
    del h0, D, Q, G, cell
    torch.cuda.empty_cache()
    return elapsed, resident, peak


def time_graphed(cfg, mode, steps, warmup):
    """The pass replayed from a HIP graph (forward-only configs: chain.capture_forward; with a backward:
    chain.capture_training, forward and backward in one graph, the loss summed eagerly after each replay), `steps`
    passes timed after `warmup`; returns elapsed s."""
    import torch
    from loopback_amd.chain import capture_forward, capture_training, make_inputs
    dev = torch.device("cuda", 0)
    h0, D, Q, G = make_inputs(cfg, dev)
    if cfg.backward:
        run = capture_training(cfg, h0, D, Q, G, mode)
    else:
        graph, _ = capture_forward(cfg, h0, D, Q, mode)
        run = graph.replay
    for _ in range(max(1, warmup)):
        run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        run()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    del run, h0, D, Q, G
    torch.cuda.empty_cache()
    return elapsed


def cpu_model() -> str | None:
    """The host CPU's model name, as lscpu reports it (else /proc/cpuinfo), with its family / model / stepping."""
    name = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        name = next((ln.split(":", 1)[1].strip() for ln in out.splitlines() if ln.startswith("Model name")), None)
    except (OSError, subprocess.SubprocessError):
        pass
    ids = {}
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ":" not in ln:
                    if ids:
                        break
                    continue
                k, v = (x.strip() for x in ln.split(":", 1))
                if k in ("model name", "cpu family", "model", "stepping") and k not in ids:
                    ids[k] = v
    except OSError:
        pass
    name = name or ids.get("model name")
    if name and all(k in ids for k in ("cpu family", "model", "stepping")):
        name += f" (family {ids['cpu family']}, model {ids['model']}, stepping {ids['stepping']})"
    return name


def _cpu_time(cfg, tokens, min_s, max_s):
    """Median seconds per oracle chain pass on `tokens` tokens (>= 5 runs after a warm-up, about min_s of work)."""
    from oracle.reference_read import run_chain
    from loopback_amd.chain import make_inputs
    h0, D, Q, G = make_inputs(cfg, "cpu", n_tok=tokens)
    run_chain(cfg.K, cfg.R, h0, D, Q, G, beta=cfg.beta, eps=cfg.eps, grad=cfg.backward)   # warm-up
    times, t_start = [], time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t_start < min_s and len(times) < 50):
        t0 = time.perf_counter()
        run_chain(cfg.K, cfg.R, h0, D, Q, G, beta=cfg.beta, eps=cfg.eps, grad=cfg.backward)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > max_s:
            break
    return statistics.median(times), len(times)


def cpu_baseline(cfg, tokens):
    """The oracle chain on the host cores on `tokens` tokens of the headline configuration (fwd+bwd), and config 1
    (the reference's CPU case) whole; tokens/s and the effective GB/s of the reference dataflow's bytes."""
    import torch
    from loopback_amd.chain import CONFIGS, algorithmic_bytes_per_token
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    med, runs = _cpu_time(cfg, tokens, 10, 30)
    e = elt_bytes(cfg.dtype)
    bpt = algorithmic_bytes_per_token(cfg.N, cfg.d, e, backward=cfg.backward)["total"]
    c1 = CONFIGS["c1"]
    med1, runs1 = _cpu_time(c1, c1.n_tok, 5, 15)
    bpt1 = algorithmic_bytes_per_token(c1.N, c1.d, 4, backward=False, dots=False)["total"]
    return {"value": tokens / med, "unit": "read-tokens/s", "cores": torch.get_num_threads(),
            "affinity_cores": cores, "cpu_model": cpu_model(), "kind": "port",
            "gbs": bpt * tokens / med / 1e9,
            "sample": f"oracle chain (restated reference read, torch CPU) {cfg.name} with T={tokens} tokens, "
                      f"{'fwd+bwd' if cfg.backward else 'fwd'}, median of {runs} runs, {med:.3f} s/run; gbs = the "
                      f"reference dataflow's {bpt} B/token x tokens/s",
            "config1": {"value": c1.n_tok / med1, "unit": "tokens/s", "gbs": bpt1 * c1.n_tok / med1 / 1e9,
                        "sample": f"oracle chain {c1.name}: d=768, K=2, R=4, T={c1.n_tok}, fp32, fwd; median of "
                                  f"{runs1} runs, {med1 * 1e3:.1f} ms/run; gbs = {bpt1} B/token (the DOTS-off form, "
                                  f"e = 4) x tokens/s"}}


def main():
    args = parse()
    if args.glue is not None:     # before the read's modules look at it
        os.environ["LOOP_DATTN_FUSE_GLUE"] = args.glue
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
    from loopback_amd.cell import fuse_glue
    from loopback_amd.chain import CONFIGS

    cfg = with_dtype(CONFIGS[args.config], args.dtype)
    dev = torch.device("cuda", 0)
    if args.graph:   # the pass replayed from HIP graphs: no Python or launch work per kernel
        elapsed = time_graphed(cfg, args.mode, args.steps, args.warmup)
        _, ref_bytes = family_bytes(cfg, args.mode)
        print(json.dumps({"metric": f"depth-read tokens/sec ({'fwd+bwd' if cfg.backward else 'fwd'}), {cfg.name}, "
                                    "HIP graph replay",
                          "value": cfg.n_tok * args.steps / elapsed, "unit": "read-tokens/s", "n_gpus": 1,
                          "steps": args.steps, "warmup": args.warmup, "ms_per_step": 1e3 * elapsed / args.steps,
                          "higher_is_better": True, "dtype": dtype_name(cfg.dtype),
                          "formula_wall_gbs": ref_bytes * args.steps / elapsed / 1e9,
                          "config": {"workload": cfg.name, "mode": args.mode, "graph": True}}), flush=True)
        return

    timer = KernelTimer()
    elapsed, resident, peak = time_chain(cfg, args.mode, args.steps, args.warmup, timer)
    ms_per_step = 1e3 * elapsed / args.steps
    ksum = timer.summary()
    fam, ref_bytes = family_bytes(cfg, args.mode)
    sv, extra_rows = reference_bytes(cfg, args.mode)
    own_bytes = sum(fam.values())
    dom = max((k for k in fam if k in ksum), key=lambda k: ksum[k]["total_ms"])
    launches = ksum[dom]["launches"]
    mean_s = ksum[dom]["mean_us"] * 1e-6
    # the reference dataflow's bytes per launch where the reference's dataflow is this kernel's (the write, the read, backward
    # pass 1); the update gradient replaces the reference's read-modify-written gradient stack, whose bytes it does
    # not move: its own compulsory bytes there
    basis = "reference" if dom in sv and dom != "dv_assemble" else "build"
    alg = (sv[dom] if basis == "reference" else fam[dom]) / launches
    achieved = alg / mean_s / 1e9
    kernel_ms = sum(v["total_ms"] for v in ksum.values())
    # the committed counter summary is of the configuration's own dtype, with the glue in the kernels
    own = cfg.dtype == CONFIGS[args.config].dtype and fuse_glue()
    table, table_label = committed_traffic_table(args.config, args.mode) if own else (None, None)
    traffic = table.get(dom) if table is not None else None
    traffic_label = table_label if traffic is not None else None
    counters = counter_chain(table, ksum) if table is not None else None

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
        "dtype": dtype_name(cfg.dtype),
        "data": "synthetic (seeded N(0,1) updates and h0, N(0,0.02^2) queries; blocks x -> x + D_s)",
        "config": {"workload": cfg.name, "d": cfg.d, "K": cfg.K, "R": cfg.R, "N": cfg.N, "tokens": cfg.n_tok,
                   "mode": args.mode, "backward": cfg.backward, "parallelism": "single GPU",
                   "glue": ("caller's glue in the read's kernels (FusedCombineStk)" if fuse_glue() else
                            "caller's glue as torch ops around FusedDattnReadStk (the reference trainer's calls)")
                   if args.mode != "list" else "caller's glue as torch ops around FusedDattnRead"},
        "roofline": {"bound": "hbm", "kernel": dom, "bytes_basis": basis, "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic, "traffic_source": traffic_label,
                     "algorithmic_bytes_per_launch": alg, "mean_launch_us": ksum[dom]["mean_us"],
                     "launches_per_step": launches,
                     "extra_rows_per_pass": extra_rows.get(dom, 0),
                     "build_bytes_per_launch": fam[dom] / launches,
                     "build_frac": fam[dom] / launches / mean_s / 1e9 / HBM_PEAK_GBS},
        "chain": {"own_bytes_per_token": own_bytes / cfg.n_tok, "kernel_ms": kernel_ms,
                  "achieved_gbs": own_bytes / (kernel_ms * 1e-3) / 1e9,
                  "reference_formula_bytes_per_token": ref_bytes / cfg.n_tok,
                  "formula_gbs": ref_bytes / (kernel_ms * 1e-3) / 1e9,
                  "formula_wall_gbs": ref_bytes / (ms_per_step * 1e-3) / 1e9,
                  # measured HBM bytes (FETCH_SIZE + WRITE_SIZE, copy-calibrated) over kernel time
                  **({"counter_gbs": counters["counter_gbs"], "counter_frac": counters["counter_gbs"] / HBM_PEAK_GBS,
                      "counter_bytes_per_pass": counters["counter_bytes_per_pass"],
                      "counter_kernel_ms": counters["counter_kernel_ms"], "counter_families": counters["families"],
                      "counter_source": table_label} if counters else {}),
                  "kernels": {k: {"launches": v["launches"], "total_ms": round(v["total_ms"], 4),
                                  "gbs": (fam[k] / (v["total_ms"] * 1e-3) / 1e9) if k in fam else None,
                                  "reference_gbs": (sv[k] / (v["total_ms"] * 1e-3) / 1e9) if k in sv else None}
                              for k, v in sorted(ksum.items())},
                  # device memory, as the reference's --bench reports it: the inputs resident before the passes,
                  # and the peak during them (the pass's stacks, saved tensors and gradients on top of the inputs)
                  "memory_gib": {"resident": resident / 2**30, "peak": peak / 2**30,
                                 "pass_peak": (peak - resident) / 2**30}},
    }
    if args.config == "c4" and not args.no_extra_configs:
        extra = {}
        for key in ("c2", "c3"):
            c = CONFIGS[key]
            _, rb = family_bytes(c, args.mode)
            for how in ("eager", "graph"):
                el = time_chain(c, args.mode, 20, 5)[0] if how == "eager" else time_graphed(c, args.mode, 20, 5)
                ms = 1e3 * el / 20
                extra[f"{key}_{how}"] = {"workload": c.name, "ms_per_step": ms, "value": c.n_tok * 20 / el,
                                         "unit": "read-tokens/s", "backward": c.backward,
                                         "formula_wall_gbs": rb / (ms * 1e-3) / 1e9,
                                         "formula_wall_frac": rb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
        # the drop-in path the reference trainer runs after the import swap: FusedDattnReadStk with the caller's
        # glue as torch ops (LOOP_DATTN_FUSE_GLUE=0), stacked with stored scores
        for key, n_steps, n_warm in (("c4", args.steps, args.warmup), ("c3", 20, 5)):
            c = CONFIGS[key]
            with env_set("LOOP_DATTN_FUSE_GLUE", "0"):
                tg = KernelTimer()
                el = time_chain(c, "scores", n_steps, n_warm, tg)[0]
                _, rb = family_bytes(c, "scores")
            ms = 1e3 * el / n_steps
            ks = tg.summary()
            lib_ms = sum(v["total_ms"] for v in ks.values())
            extra[f"{key}_torch_glue"] = {
                "workload": c.name, "path": "FusedDattnReadStk with the caller's glue as torch ops "
                                            "(LOOP_DATTN_FUSE_GLUE=0, stored scores)",
                "ms_per_step": ms, "value": c.n_tok * n_steps / el, "unit": "read-tokens/s", "backward": c.backward,
                "steps": n_steps, "warmup": n_warm,
                "formula_wall_gbs": rb / (ms * 1e-3) / 1e9, "formula_wall_frac": rb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                "library_kernel_ms": lib_ms, "other_ms": ms - lib_ms,
                "kernels_ms": {k: round(v["total_ms"], 4) for k, v in sorted(ks.items())}}
        # config 2 runs both score modes: the table stored at the write (above) and the reads forming the scores
        # as they stream (LOOP_DATTN_DOTS=0, the stack without a score table)
        c = CONFIGS["c2"]
        _, rb = family_bytes(c, "stack")
        el = time_chain(c, "stack", 20, 5)[0]
        extra["c2_dots_off_eager"] = {"workload": c.name + " DOTS off", "ms_per_step": 1e3 * el / 20,
                                      "value": c.n_tok * 20 / el, "unit": "read-tokens/s", "backward": False,
                                      "formula_wall_gbs": rb / (el / 20) / 1e9,
                                      "formula_wall_frac": rb / (el / 20) / 1e9 / HBM_PEAK_GBS}
        from loopback_amd import lm
        for key, residual in (("c5_lm", "delta_attnres"), ("c5_lm_plain_loop", "none")):
            rec = lm.time_training(10, 3, residual=residual)
            extra[key] = {"workload": f"LM training step {rec['config']['topology']} d=768 seq 2048 x batch 8 "
                                      f"vocab 32000 ({'Loopback read' if residual != 'none' else 'Plain Loop'})",
                          "ms_per_step": rec["ms_per_step"], "value": rec["value"], "unit": rec["unit"]}
        line["configs"] = extra
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(cfg, args.cpu_tokens)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
