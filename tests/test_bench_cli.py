"""bench.py's contract on the CPU: one GPU only (a clear refusal above one,
before anything touches a GPU)."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_world_size_above_one_is_refused():
    env = dict(os.environ, WORLD_SIZE="2")
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")], capture_output=True, text=True,
                       timeout=120, cwd=ROOT, env=env)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_rotation_rows_hold_whole_matrices():
    """Every format's rotation row holds one whole matrix (the planes layout:
    code plane, then scale plane), so the streaming-read yardstick, which
    reads one matrix's bytes from each row start, stays inside the row -- and,
    for the last row, inside the allocation."""
    sys.path.insert(0, ROOT)
    import bench
    for fmt in ("q4_k", "q4_0", "planes"):
        for N, K in ((5120, 5120), (17408, 5120), (5120, 17408), (7168, 5120)):
            row, w0, wn, a0, an = bench.row_layout(fmt, N, K)
            assert row == N * K * 9 // 16
            assert (N * K * 9 // 16) // 16 * 16 <= row
            assert w0 == 0 and w0 + wn <= row
            if fmt == "planes":
                assert wn == N * K // 2 and an == N * K // 16 and a0 == wn and a0 + an == row
                assert a0 % 256 == 0 and row % 256 == 0       # the scale plane 16-byte aligned in every row
            else:
                assert wn == row and a0 is None


def test_trace_summary_groups_runs_and_passes(tmp_path):
    """--trace-summary on a synthetic kernel trace: runs of one kernel, passes
    of --trace-pass dispatches, dispatch means and per-pass spans."""
    import csv
    path = tmp_path / "kt.csv"
    cols = ["Kind", "Kernel_Name", "Start_Timestamp", "End_Timestamp"]
    t, rows = 1000, []
    for name, dur, gap, n in (("void bf::k_a<1, true>(int, float*)", 600, 100, 8),
                              ("void other_kernel(int)", 50, 0, 1),
                              ("void bf::k_b<2>(int)", 900, 0, 4)):
        for _ in range(n):
            rows.append({"Kind": "KERNEL_DISPATCH", "Kernel_Name": name, "Start_Timestamp": t,
                         "End_Timestamp": t + dur})
            t += dur + gap
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=cols)
        w.writeheader()
        w.writerows(rows)
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--trace-summary", str(path),
                        "--trace-pass", "4", "--trace-labels", "a,b"], capture_output=True, text=True, timeout=120,
                       cwd=ROOT)
    assert r.returncode == 0, r.stderr
    import json
    rec = json.loads(r.stdout)
    assert rec["a"]["kernel"] == "bf::k_a<1, true>" and rec["a"]["dispatches"] == 8 and rec["a"]["passes"] == 2
    assert rec["a"]["us_dispatch_mean"] == 0.6
    # a pass of 4 dispatches spans 4 * 600 + 3 * 100 ns
    assert abs(rec["a"]["us_span_per_launch_median"] - (4 * 600 + 3 * 100) / 4 / 1000) < 1e-9
    assert rec["b"]["passes"] == 1 and rec["b"]["us_gap_median"] == 0.0


def test_roofline_basis_is_the_committed_kernel_time(tmp_path, monkeypatch):
    """roofline.frac = algorithmic bytes / the committed per-launch time / peak;
    this run's figures sit beside it; without an entry the basis is this run's."""
    sys.path.insert(0, ROOT)
    import bench
    alg = 14_776_320
    committed = bench.kernel_time_from_profiles("q4_k_5120_m1")
    r = bench.roofline_record("q4_k_5120_m1", alg, 6.5e-6)
    assert r["us_per_launch_events"] == 6.5 and abs(r["frac_events"] - alg / 6.5e-6 / 8e12) < 1e-4
    if committed:
        assert r["us_per_launch"] == round(committed["us_per_launch"], 4)
        assert abs(r["frac"] - alg / (committed["us_per_launch"] * 1e-6) / 8e12) < 1e-4
        assert r["duration_source"].startswith("profiles/kernel_time.json")
    r = bench.roofline_record("no_such_key", alg, 6.5e-6)
    assert r["us_per_launch"] == 6.5 and r["frac"] == r["frac_events"] and "this run" in r["duration_source"]
    # the writer keeps other entries and stores the best launch mode per batch size
    path = tmp_path / "kt.json"
    path.write_text('{"other": {"us_per_launch": 1.0}}')
    recs = [{"M": 1, "us_per_gemm": 6.2, "launch": "stream", "gemms_timed": 72, "ms_per_pass": 0.4464},
            {"M": 1, "us_per_gemm": 6.1, "launch": "graph", "gemms_timed": 72, "ms_per_pass": 0.4392}]
    bench.write_kernel_time(str(path), "q4_k", 5120, 5120, recs, [1], ["--no-cpu"])
    import json
    d = json.loads(path.read_text())
    assert d["other"]["us_per_launch"] == 1.0
    assert d["q4_k_5120_m1"]["us_per_launch"] == 6.1 and d["q4_k_5120_m1"]["launch"] == "graph"
    # runs of one library build keep the best time and count the runs; a new build starts over
    monkeypatch.setattr(bench, "library_digest", lambda: "aaaa")
    path.write_text("{}")
    for us in (6.3, 6.1, 6.2):
        bench.write_kernel_time(str(path), "q4_k", 5120, 5120, [dict(recs[0], us_per_gemm=us)], [1], ["--no-cpu"])
    e = json.loads(path.read_text())["q4_k_5120_m1"]
    assert e["us_per_launch"] == 6.1 and e["runs"] == 3 and e["lib_sha16"] == "aaaa"
    monkeypatch.setattr(bench, "library_digest", lambda: "bbbb")
    bench.write_kernel_time(str(path), "q4_k", 5120, 5120, [dict(recs[0], us_per_gemm=6.4)], [1], ["--no-cpu"])
    e = json.loads(path.read_text())["q4_k_5120_m1"]
    assert e["us_per_launch"] == 6.4 and e["runs"] == 1 and e["lib_sha16"] == "bbbb"


def test_counter_summary_means_per_dispatch(tmp_path):
    """--counter-summary: a dispatch's rows of one counter summed, then the
    mean over the kernel's dispatches; other processes' kernels left out."""
    import csv
    import json
    path = tmp_path / "pmc.csv"
    cols = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
    rows = []
    for d, (k, vals) in enumerate((("void bf::k_x<1>(int)", (10, 20)), ("void bf::k_x<1>(int)", (30, 40)),
                                   ("(anonymous namespace)::k_stream_copy(int)", (5,)), ("void at::foo(int)", (99,)))):
        for v in vals:
            rows.append({"Dispatch_Id": d, "Kernel_Name": k, "Counter_Name": "FETCH_SIZE", "Counter_Value": v})
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=cols)
        w.writeheader()
        w.writerows(rows)
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--counter-summary", str(path)],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 0, r.stderr
    rec = json.loads(r.stdout)
    assert rec["bf::k_x<1>"] == {"dispatches": 2, "FETCH_SIZE": 50.0}
    assert rec["(anonymous namespace)::k_stream_copy"]["FETCH_SIZE"] == 5.0 and "at::foo" not in rec
