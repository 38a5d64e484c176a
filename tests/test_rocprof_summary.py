"""The profile summaries' arithmetic (loopback_amd/rocprof_summary.py) on small synthetic rocprofv3 outputs: the chain
passes are split at each pass's k_split_queries launch and the last complete one is summarized (the final pass runs
into the program's end), a counter run's last pass is summed per kernel family, the copy calibration scales the
counters so that a 1 GiB copy reads as 1 GiB, and the traffic file records per-launch bytes from those."""
import csv
import json
import os

import pytest

from loopback_amd import rocprof_summary as RS

# one chain pass: (kernel, duration ns); the torch add stands for the caller's ops
PASS = [("k_split_queries(...)", 4_000), ("k_write_rows<unsigned short, 1>(...)", 37_000),
        ("at::native::vectorized_elementwise_kernel<8, CUDAFunctor_add>", 30_000),
        ("k_write_rows<unsigned short, 2>(...)", 39_000), ("k_read_fwd<unsigned short, 4, false, true, 512>(...)", 210_000),
        ("k_bwd1<unsigned short, 4, 1>(...)", 200_000), ("k_dv_assemble<unsigned short, 2, true, false>(...)", 205_000),
        ("k_dv_assemble<unsigned short, 2, true, false>(...)", 207_000)]


def _write_csv(path, fields, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        w.writerows(rows)


def _trace(path, passes=3, scale=1):
    rows, t = [], 1_000_000
    for p in range(passes):
        for name, ns in PASS:
            rows.append({"Kernel_Name": name, "Start_Timestamp": t, "End_Timestamp": t + ns * scale * (p + 1)})
            t += ns * scale * (p + 1) + 1_000
    _write_csv(path, ["Kernel_Name", "Start_Timestamp", "End_Timestamp"], rows)


def _counter(path, counter, kib_of, passes=2):
    rows, disp = [], 0
    for _ in range(passes):
        for name, _ns in PASS:
            disp += 1
            rows.append({"Dispatch_Id": disp, "Kernel_Name": name, "Counter_Name": counter,
                         "Counter_Value": kib_of(name)})
    _write_csv(path, ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"], rows)


def test_last_complete_pass_and_its_span(tmp_path):
    p = tmp_path / "kt.csv"
    _trace(p)
    fams, span_ms = RS.trace_pass(str(p))
    # the second pass (durations doubled): the families' launches and time
    assert fams["write_dots"] == [2, pytest.approx(2 * (37 + 39))]
    assert fams["dv_assemble"] == [2, pytest.approx(2 * (205 + 207))]
    assert fams["read_fwd"] == [1, pytest.approx(420.0)]
    assert fams["torch / runtime"] == [1, pytest.approx(60.0)]
    assert span_ms == pytest.approx((2 * sum(ns for _, ns in PASS) + len(PASS) * 1_000) / 1e6)


def test_counter_pass_and_calibration(tmp_path):
    cf = tmp_path / "pf.csv"
    _counter(cf, "FETCH_SIZE", lambda name: 1000.0 if "dv_assemble" in name else 10.0)
    out = RS.counter_pass(str(cf), "FETCH_SIZE")
    assert out["dv_assemble"] == [2, 2000.0]   # the last pass alone
    cal = tmp_path / "cf.csv"
    _write_csv(cal, ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"],
               [{"Dispatch_Id": 1, "Kernel_Name": "__amd_rocclr_copyBuffer", "Counter_Name": "FETCH_SIZE",
                 "Counter_Value": 524288.0}])
    assert RS.calibration(str(cal), "FETCH_SIZE") == pytest.approx(2.0)   # 1 GiB read as 512 MiB


def test_traffic_file_per_launch_bytes(tmp_path):
    kt, pf, pw, cf, cw = (tmp_path / f"{n}.csv" for n in ("kt", "pf", "pw", "cf", "cw"))
    _trace(kt)
    _write_csv(tmp_path / "st.csv", ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage"],
               [{"Name": "k_bwd1<unsigned short, 4, 1>(...)", "Calls": 3, "TotalDurationNs": 600_000,
                 "AverageNs": 200_000, "Percentage": 100.0}])
    _counter(pf, "FETCH_SIZE", lambda name: 500_000.0 if "read_fwd" in name else 1.0)
    _counter(pw, "WRITE_SIZE", lambda name: 100_000.0 if "read_fwd" in name else 1.0)
    for path, counter, kib in ((cf, "FETCH_SIZE", 524288.0), (cw, "WRITE_SIZE", 1048576.0)):
        _write_csv(path, ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"],
                   [{"Dispatch_Id": 1, "Kernel_Name": "__amd_rocclr_copyBuffer", "Counter_Name": counter,
                     "Counter_Value": kib}])
    out = tmp_path / "profiles"
    out.mkdir()
    RS.main(["--trace", str(kt), "--stats", str(tmp_path / "st.csv"), "--fetch", str(pf), "--write", str(pw),
             "--calib-fetch", str(cf), "--calib-write", str(cw), "--config", "c4", "--mode", "scores",
             "--out", str(out), "--commit", "abc1234"])
    tr = json.loads((out / "traffic_chain_c4.txt").read_text())
    assert tr["fetch_scale"] == pytest.approx(2.0) and tr["write_scale"] == pytest.approx(1.0)
    # one read_fwd launch: 500000 KiB fetched x 2 + 100000 KiB written x 1
    assert tr["hbm_bytes_per_launch"]["read_fwd"] == pytest.approx((500_000 * 2 + 100_000) * 1024)
    assert tr["commit"] == "abc1234" and tr["dtype"] == "bf16"
    assert os.path.exists(out / "kernels_chain_c4.md") and os.path.exists(out / "traffic_chain_c4.md")
    assert tr["glue"] == "1"


def test_torch_glue_summaries_are_named_apart(tmp_path):
    """--glue 0 (a profile of bench.py --glue 0) writes *_torchglue summaries, counted with the torch-glue path's
    bytes (no iteration-end h0 rows, no blend sum), and leaves the process's environment as it was."""
    kt, pf, pw, cf, cw = (tmp_path / f"{n}.csv" for n in ("kt", "pf", "pw", "cf", "cw"))
    _trace(kt)
    _counter(pf, "FETCH_SIZE", lambda name: 10.0)
    _counter(pw, "WRITE_SIZE", lambda name: 10.0)
    for path, counter, kib in ((cf, "FETCH_SIZE", 524288.0), (cw, "WRITE_SIZE", 1048576.0)):
        _write_csv(path, ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"],
                   [{"Dispatch_Id": 1, "Kernel_Name": "__amd_rocclr_copyBuffer", "Counter_Name": counter,
                     "Counter_Value": kib}])
    out = tmp_path / "profiles"
    out.mkdir()
    before = os.environ.get("LOOP_DATTN_FUSE_GLUE")
    RS.main(["--trace", str(kt), "--fetch", str(pf), "--write", str(pw), "--calib-fetch", str(cf),
             "--calib-write", str(cw), "--config", "c4", "--mode", "scores", "--glue", "0", "--out", str(out)])
    assert os.environ.get("LOOP_DATTN_FUSE_GLUE") == before
    assert json.loads((out / "traffic_chain_c4_torchglue.txt").read_text())["glue"] == "0"
    text = (out / "kernels_chain_c4_torchglue.md").read_text()
    assert "torch ops" in text
    # the read forward's bytes without the blend's h0 rows: sum_s (n + 2) rows of 64 MiB
    N, row = 32, 2 * 2048 * 16384
    reads = (N * (N + 1) // 2 - 1 + 2 * (N - 1)) * row
    assert f"| {reads / 1e9:.2f} |" in text


def test_bench_counter_chain_arithmetic():
    """bench.counter_chain: measured bytes per launch x this pass's launches, over the same families' kernel time;
    families the table lacks (or the pass lacks) are left out of both sums."""
    import bench
    table = {"read_fwd": 2e9, "read_bwd1": 1e9, "blend_sum": 5e8}
    ksum = {"read_fwd": {"launches": 3, "total_ms": 1.0}, "read_bwd1": {"launches": 2, "total_ms": 0.5},
            "reduce_rows": {"launches": 1, "total_ms": 0.25}}
    c = bench.counter_chain(table, ksum)
    assert c["families"] == ["read_bwd1", "read_fwd"]
    assert c["counter_bytes_per_pass"] == pytest.approx(3 * 2e9 + 2 * 1e9)
    assert c["counter_kernel_ms"] == pytest.approx(1.5)
    assert c["counter_gbs"] == pytest.approx(8e9 / 1.5e-3 / 1e9)
    assert bench.counter_chain({"x": 1.0}, ksum) is None


def test_compare_pass_timelines(tmp_path):
    """--compare: the last complete pass of each trace -- its kernel time, span, idle time between its kernels and
    before the next pass -- from synthetic traces whose timings are known."""
    kt1, kt2 = tmp_path / "e.csv", tmp_path / "g.csv"
    _trace(kt1)                    # 1 us between kernels
    _trace(kt2, scale=2)
    t = RS.pass_timeline(str(kt1))
    ns = sum(ns for _, ns in PASS)
    assert t["kernels"] == len(PASS)
    assert t["busy_us"] == pytest.approx(2 * ns / 1e3)        # the second of three passes runs at twice the time
    assert t["gaps_us"] == pytest.approx((len(PASS) - 1) * 1.0)
    assert t["to_next_us"] == pytest.approx(1.0)
    assert t["span_us"] == pytest.approx(t["busy_us"] + t["gaps_us"])
    out = tmp_path / "profiles"
    out.mkdir()
    RS.main(["--config", "c3", "--compare", str(kt1), str(kt2), "--name", "cmp", "--out", str(out)])
    text = (out / "cmp.md").read_text()
    assert "| eager | 8 |" in text and "| graph replay | 8 |" in text
