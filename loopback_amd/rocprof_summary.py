"""Summaries of rocprofv3 output for the headline chain: per-kernel time of one pass (kernel trace) and HBM bytes per
launch (FETCH_SIZE / WRITE_SIZE counter passes, scaled by what the same counters read for a device-to-device copy of
known size). Writes the markdown tables kept with the profiles and the per-launch traffic figure bench.py reports.

    python -m loopback_amd.rocprof_summary --trace prof/kt/kt_kernel_trace.csv \\
        --stats prof/kt/kt_kernel_stats.csv --fetch prof/pf/pf_counter_collection.csv \\
        --write prof/pw/pw_counter_collection.csv \\
        --calib-fetch prof/cf/cf_counter_collection.csv --calib-write prof/cw/cw_counter_collection.csv \\
        --config c4 --mode scores --out profiles

Run it in the job that profiled (the traffic summary records the sha256 of the kernel source it finds, which bench.py
compares with its own). The passes are split at the one k_split_queries launch each chain pass starts with (modes without stored scores: at
the first forward kernel of the library after a backward one); the last complete pass of the trace and the last
pass of each counter run are the ones summarized. `--stats-only NAME` summarizes the --stats
output of any run (the LM step) into profiles/NAME.md.
"""
from __future__ import annotations

import argparse
import csv
import json
import os
import sys

FAMILIES = [("k_read_fwd", "read_fwd"), ("k_read_online", "read_fwd_online"), ("k_bwd1", "read_bwd1"), ("k_dv_assemble", "dv_assemble"),
            ("k_write_mfma", "write_dots"), ("k_write_rows", "write_dots"), ("k_write_dots", "write_dots"), ("k_dots", "dots_online"),
            ("k_reduce_rows", "reduce_rows"), ("k_split_queries", "split_queries"), ("k_rstd", "rstd"),
            ("k_bwd2_list", "read_bwd2_list"), ("k_blend_sum", "blend_sum")]
COPY_BYTES = 1 << 30   # bench.py --copy-calibration copies 1 GiB


def family(name: str) -> str:
    for key, fam in FAMILIES:
        if key in name:
            return fam
    return "torch / runtime"


def _rows(path):
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


FWD_KERNELS = ("k_split_queries", "k_write_mfma", "k_write_rows", "k_write_dots", "k_rstd_fwd", "k_read_fwd", "k_read_online", "k_dots")
BWD_KERNELS = ("k_bwd1", "k_dv_assemble", "k_reduce_rows", "k_blend_sum", "k_bwd2_list", "k_rstd_bwd")


def _passes(rows, key="Start_Timestamp", n_steps=None):
    """The rows of each chain pass, in launch order. With stored scores a pass starts at its k_split_queries launch
    (the stack's queries); otherwise at the first forward kernel of the library after a backward one; a forward-only
    chain without stored scores (no backward kernels) at every n_steps-th write (a pass writes n_steps updates)."""
    rows = sorted(rows, key=lambda r: int(r[key]))
    starts = [i for i, r in enumerate(rows) if "k_split_queries" in r["Kernel_Name"]]
    if not starts:
        prev = None
        for i, r in enumerate(rows):
            name = r["Kernel_Name"]
            kind = "f" if any(k in name for k in FWD_KERNELS) else "b" if any(k in name for k in BWD_KERNELS) else None
            if kind == "f" and prev != "f":
                starts.append(i)
            prev = kind or prev
        if len(starts) < 2 and n_steps:
            starts = [i for i, r in enumerate(rows) if family(r["Kernel_Name"]) == "write_dots"][::n_steps]
    return [rows[a:b] for a, b in zip(starts, starts[1:] + [len(rows)])]


def trace_pass(path, n_steps=None):
    """Per-family launches and GPU time of the last complete pass of a kernel trace; also the pass's span."""
    passes = _passes(_rows(path), n_steps=n_steps)
    if len(passes) < 2:
        raise SystemExit("kernel trace: need at least two chain passes")
    p = passes[-2]   # the last complete pass (the final one runs into the end of the program)
    out = {}
    for r in p:
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        t = out.setdefault(family(r["Kernel_Name"]), [0, 0.0])
        t[0] += 1
        t[1] += us
    nxt = passes[-1][0]
    span_ms = (int(nxt["Start_Timestamp"]) - int(p[0]["Start_Timestamp"])) / 1e6
    return out, span_ms


def pass_timeline(path, n_steps=None):
    """The last complete pass of a kernel trace as a timeline: kernels, kernel time (us), the span from its first
    kernel's start to its last kernel's end, the idle time between its kernels, and the idle time from its last kernel
    to the next pass's first (all in us)."""
    passes = _passes(_rows(path), n_steps=n_steps)
    if len(passes) < 2:
        raise SystemExit("kernel trace: need at least two chain passes")
    p, nxt = passes[-2], passes[-1][0]
    ts = lambda r, k: int(r[k])
    busy = sum(ts(r, "End_Timestamp") - ts(r, "Start_Timestamp") for r in p) / 1e3
    span = (ts(p[-1], "End_Timestamp") - ts(p[0], "Start_Timestamp")) / 1e3
    gaps = sum(max(0, ts(b, "Start_Timestamp") - ts(a, "End_Timestamp")) for a, b in zip(p, p[1:])) / 1e3
    tail = (ts(nxt, "Start_Timestamp") - ts(p[-1], "End_Timestamp")) / 1e3
    return {"kernels": len(p), "busy_us": busy, "span_us": span, "gaps_us": gaps, "to_next_us": tail,
            "period_us": (ts(nxt, "Start_Timestamp") - ts(p[0], "Start_Timestamp")) / 1e3}


def counter_pass(path, counter, n_steps=None):
    """Per-family launches and counter total (KiB) of the last pass of a counter run."""
    rows = [r for r in _rows(path) if r["Counter_Name"] == counter]
    # one row per dispatch per counter
    p = _passes(rows, key="Dispatch_Id", n_steps=n_steps)[-1]
    out = {}
    for r in p:
        t = out.setdefault(family(r["Kernel_Name"]), [0, 0.0])
        t[0] += 1
        t[1] += float(r["Counter_Value"])
    return out


def calibration(path, counter):
    rows = [r for r in _rows(path) if r["Counter_Name"] == counter and "copyBuffer" in r["Kernel_Name"]]
    if not rows:
        raise SystemExit(f"calibration: no copy kernel in {path}")
    kib = max(float(r["Counter_Value"]) for r in rows)
    return (COPY_BYTES / 1024) / kib


def stats_table(path, top):
    """rocprofv3's --stats kernel summary, the `top` kernels by total time, names shortened."""
    st = sorted(_rows(path), key=lambda r: -float(r["TotalDurationNs"]))
    total = sum(float(r["TotalDurationNs"]) for r in st)
    lines = [f"rocprofv3 --stats over the whole run ({total / 1e6:.1f} ms of kernel time in all; names shortened):",
             "", "| kernel | calls | total ms | average us | % |", "|---|---|---|---|---|"]
    for r in st[:top]:
        name = r["Name"].replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0][:80]
        lines.append(f"| `{name}` | {r['Calls']} | {float(r['TotalDurationNs']) / 1e6:.2f} | "
                     f"{float(r['AverageNs']) / 1e3:.1f} | {r['Percentage']} |")
    fams = {}
    for r in st:   # this library's kernels, whether or not they made the table
        fam = family(r["Name"])
        if fam != "torch / runtime":
            f = fams.setdefault(fam, [0, 0.0])
            f[0] += int(r["Calls"])
            f[1] += float(r["TotalDurationNs"])
    if fams:
        lib = sum(v[1] for v in fams.values())
        lines += ["", f"This library's kernels: {lib / 1e6:.2f} ms of the {total / 1e6:.1f} ms "
                      f"({100 * lib / total:.1f} %).", "", "| kernel family | calls | total ms |", "|---|---|---|"]
        for fam, (n, ns) in sorted(fams.items(), key=lambda x: -x[1][1]):
            lines.append(f"| `{fam}` | {n} | {ns / 1e6:.2f} |")
    return lines


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--trace", default=None)
    ap.add_argument("--stats", default=None, help="the --stats kernel summary of the same trace run")
    ap.add_argument("--fetch", default=None)
    ap.add_argument("--write", default=None)
    ap.add_argument("--calib-fetch", default=None)
    ap.add_argument("--calib-write", default=None)
    ap.add_argument("--stats-only", default=None, metavar="NAME",
                    help="write only the --stats table, as profiles/NAME.md (any program, e.g. the LM step)")
    ap.add_argument("--title", default="", help="heading of a --stats-only summary")
    ap.add_argument("--compare", nargs=2, default=None, metavar=("EAGER", "REPLAY"),
                    help="two kernel traces of the same configuration (eager, replayed from a HIP graph): writes "
                         "profiles/NAME.md (--name) with each one's pass timeline")
    ap.add_argument("--name", default=None, help="file name of a --compare summary")
    ap.add_argument("--config", default="c4")
    ap.add_argument("--mode", default="scores")
    ap.add_argument("--dtype", default=None, choices=["bf16", "fp16", "fp32"],
                    help="the update dtype the run used (bench.py --dtype), when not the configuration's own")
    ap.add_argument("--glue", default="1", choices=["0", "1"],
                    help="LOOP_DATTN_FUSE_GLUE of the profiled run (bench.py --glue): 0 names the summaries "
                         "*_torchglue and counts the bytes of the torch-glue path")
    ap.add_argument("--out", default="profiles")
    ap.add_argument("--commands", default="", help="the commands that produced the inputs (quoted into the summaries)")
    ap.add_argument("--commit", default=None, help="the commit the profiled tree was taken from (recorded as given)")
    a = ap.parse_args(argv)
    if a.compare:
        root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
        sys.path.insert(0, root)
        from loopback_amd.chain import CONFIGS
        cfg = CONFIGS[a.config]
        lines = [f"# {a.title or 'Eager against HIP-graph replay'}: config {a.config} ({cfg.name})", ""]
        if a.commands:
            lines += ["Commands:", "", *["    " + c for c in a.commands.split(";;")], ""]
        lines += ["The last complete pass of each trace (us): kernel time, the span from its first kernel's start to its "
                  "last kernel's end, the idle time between its kernels, the idle time before the next pass's first "
                  "kernel, and the period between pass starts. The eager trace's idle time is the profiler's slow-down "
                  "of the host's launches.", "",
                  "| run | kernels | kernel time | span | idle between kernels | idle before the next pass | period |",
                  "|---|---|---|---|---|---|---|"]
        for label, path in zip(("eager", "graph replay"), a.compare):
            t = pass_timeline(path, cfg.N)
            lines.append(f"| {label} | {t['kernels']} | {t['busy_us']:.1f} | {t['span_us']:.1f} | {t['gaps_us']:.1f} | "
                         f"{t['to_next_us']:.1f} | {t['period_us']:.1f} |")
        with open(os.path.join(a.out, f"{a.name or 'graph_replay_' + a.config}.md"), "w") as f:
            f.write("\n".join(lines) + "\n")
        return
    if a.stats_only:
        lines = [f"# {a.title or a.stats_only}", ""]
        if a.commands:
            lines += ["Commands:", "", *["    " + c for c in a.commands.split(";;")], ""]
        lines += stats_table(a.stats, 20)
        with open(os.path.join(a.out, f"{a.stats_only}.md"), "w") as f:
            f.write("\n".join(lines) + "\n")
        return
    if a.trace is None:
        ap.error("--trace is required")
    counters = [a.fetch, a.write, a.calib_fetch, a.calib_write]
    if any(c is not None for c in counters) and not all(c is not None for c in counters):
        ap.error("--fetch, --write, --calib-fetch and --calib-write go together (or none: the kernel table alone)")

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    sys.path.insert(0, root)
    import bench   # the byte model the bench line uses
    from loopback_amd.chain import CONFIGS
    cfg = bench.with_dtype(CONFIGS[a.config], a.dtype)
    with bench.env_set("LOOP_DATTN_FUSE_GLUE", a.glue):   # the byte model of the profiled run's glue setting
        fam_bytes, _ = bench.family_bytes(cfg, a.mode)
        sv_bytes, _ = bench.reference_bytes(cfg, a.mode)

    kt, span_ms = trace_pass(a.trace, cfg.N)

    # the headline mode and the configuration's own dtype keep the plain name
    tag = a.config + ("" if a.mode == "scores" else f"_{a.mode}") + \
        ("" if cfg.dtype == CONFIGS[a.config].dtype else f"_{bench.dtype_name(cfg.dtype)}") + \
        ("" if a.glue == "1" or a.mode == "list" else "_torchglue")
    busy = sum(v[1] for v in kt.values()) / 1e3
    glue = "" if a.mode == "list" else (", the caller's glue as torch ops (LOOP_DATTN_FUSE_GLUE=0)" if a.glue == "0"
                                        else ", the caller's glue in the read's kernels")
    lines = [f"# Kernel time per chain pass: config {a.config} ({cfg.name}), mode {a.mode}{glue}", ""]
    if a.commands:
        lines += ["Commands:", "", *["    " + c for c in a.commands.split(";;")], ""]
    lines += [f"One pass (the last complete one of the trace): span {span_ms:.2f} ms between pass starts, "
              f"{busy:.2f} ms of kernel time.", "",
              "Algorithmic GB: this build's compulsory rows (bench.py `family_bytes`); reference GB: the "
              "reference dataflow's rows for the same work (bench.py `reference_bytes`), each over the family's "
              "kernel time. The reference's figure for the update gradient counts the reference's read-modify-written gradient "
              "stack, bytes this kernel does not move; the last column is the bench line's roofline fraction: the "
              "reference's bytes where its dataflow is the kernel's, the kernel's own for the update gradient, against "
              "8000 GB/s.", "",
              "| kernel family | launches | total ms | mean us | algorithmic GB | GB/s | reference GB | GB/s (reference) "
              "| of peak (roofline bytes) |", "|---|---|---|---|---|---|---|---|---|"]
    for famname, (n, us) in sorted(kt.items(), key=lambda x: -x[1][1]):
        ab, sb = fam_bytes.get(famname), sv_bytes.get(famname)
        cols = [f"{ab / 1e9:.2f}", f"{ab / (us * 1e-6) / 1e9:.0f}"] if ab else ["-", "-"]
        rb = ab if famname == "dv_assemble" else sb
        cols += ([f"{sb / 1e9:.2f}", f"{sb / (us * 1e-6) / 1e9:.0f}", f"{rb / (us * 1e-6) / 1e9 / 8000:.3f}"]
                 if sb else ["-", "-", "-"])
        lines.append(f"| `{famname}` | {n} | {us / 1e3:.3f} | {us / n:.1f} | " + " | ".join(cols) + " |")
    if a.stats:   # rocprofv3's own per-kernel summary over the whole run (warm-up and timed passes)
        lines += [""] + stats_table(a.stats, 12)
    with open(os.path.join(a.out, f"kernels_chain_{tag}.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    if a.fetch is None:
        return
    fetch = counter_pass(a.fetch, "FETCH_SIZE", cfg.N)
    write = counter_pass(a.write, "WRITE_SIZE", cfg.N)
    fs = calibration(a.calib_fetch, "FETCH_SIZE")
    ws = calibration(a.calib_write, "WRITE_SIZE")

    per_launch = {}
    lines = [f"# HBM traffic per kernel: config {a.config} ({cfg.name}), mode {a.mode}{glue}, one pass", ""]
    if a.commands:
        lines += ["Commands:", "", *["    " + c for c in a.commands.split(";;")], ""]
    lines += [f"Calibration: a 1 GiB device-to-device copy reads FETCH_SIZE = {(COPY_BYTES / 1024) / fs:.0f} KiB and "
              f"WRITE_SIZE = {(COPY_BYTES / 1024) / ws:.0f} KiB, so FETCH_SIZE is scaled by {fs:.3f} and WRITE_SIZE "
              f"by {ws:.3f}.", "",
              "| kernel | launches | fetched GB (scaled) | written GB (scaled) | algorithmic GB | measured / algorithmic "
              "| HBM bytes per launch |", "|---|---|---|---|---|---|---|"]
    for famname in sorted(fam_bytes, key=lambda k: -fam_bytes[k]):
        if famname not in fetch:
            continue
        n = fetch[famname][0]
        fb = fetch[famname][1] * 1024 * fs
        wb = write.get(famname, [0, 0.0])[1] * 1024 * ws
        per_launch[famname] = (fb + wb) / n
        lines.append(f"| `{famname}` | {n} | {fb / 1e9:.2f} | {wb / 1e9:.2f} | {fam_bytes[famname] / 1e9:.2f} | "
                     f"{(fb + wb) / fam_bytes[famname]:.3f} | {per_launch[famname]:.0f} |")
    lines += ["", "Algorithmic bytes: the compulsory rows of each kernel family (bench.py `family_bytes`); per-(token, "
              "source) fp32 scalars are not counted, which is most of the excess."]
    with open(os.path.join(a.out, f"traffic_chain_{tag}.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    with open(os.path.join(a.out, f"traffic_chain_{tag}.txt"), "w") as f:
        json.dump({"config": a.config, "mode": a.mode, "glue": a.glue, "dtype": bench.dtype_name(cfg.dtype),
                   "source": f"profiles/traffic_chain_{tag}.md (commands and calibration there)",
                   # the kernel source the counters were read on (this tool runs in the same job as the profile)
                   "source_sha256": bench.source_sha256(), "commit": a.commit,
                   "fetch_scale": fs, "write_scale": ws, "hbm_bytes_per_launch": per_launch}, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
