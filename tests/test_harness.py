"""Harness behaviour on the CPU: gate, report text, persistence, CLI."""
import io
import json
import re
import subprocess
import sys
from contextlib import redirect_stdout

import numpy as np
import pytest

from metalbench_amd import harness, roofline
from metalbench_amd import helpers as H

REPO = H.REPO_ROOT

# Regexes of the reference's report consumers, kept verbatim in meaning:
# agent_steel/profiler/bench_runner.py:71-83 and tests/metalbench/test_bench_accuracy_all.py:32.
RX = {
    "correct": re.compile(r"correctness\s+:\s*(✓\s*correct|✗\s*incorrect).*?max_err=([\d.eE+-]+)"),
    "speedup": re.compile(r"speedup\s+:\s*([\d.eE+-]+)×"),
    "kernel": re.compile(r"kernel\s+:\s*([\d.eE+-]+)\s*ms\s+\(min\s*([\d.eE+-]+),\s*mean\s*([\d.eE+-]+),\s*n=\d+\)"),
    "mlx": re.compile(r"mlx\s+ref\s+:\s*([\d.eE+-]+)\s*ms"),
    "gflops": re.compile(r"compute\s+:\s*([\d.eE+-]+)\s*GFLOPS"),
    "gbps": re.compile(r"bandwidth\s+:\s*([\d.eE+-]+)\s*GB/s"),
    "ai": re.compile(r"arith\s+int\.\s*:\s*([\d.eE+-]+)"),
    "stability": re.compile(r"stability\s+:\s*([\d.eE+-]+)"),
    "occupancy": re.compile(r"occupancy\s+:\s*tg_mem=(\d+)\s*KB\s+max_thr/tg=(\d+)"),
    "accuracy": re.compile(r"correctness\s+:\s*(✓|✗).*?max_err=([\d.eE+-]+)"),
}


def _fake_result(correct=True, median=0.128):
    chip = {"type": "gfx950", "name": "AMD Instinct MI355X", "bucket": "amd-instinct-mi355x",
            "cpu_cores": 16, "gpu_cores": 256, "ram_bytes": 3e11}
    k_t = {"min_ms": 0.12, "median_ms": median, "mean_ms": 0.13, "iters": 200}
    r_t = {"min_ms": 70.0, "median_ms": 74.5, "mean_ms": 74.6, "iters": 5, "label": "cpu spec"}
    m = {"speedup": 74.5 / median, "gflops": 0.0, "gbps": 536870912 / (median * 1e-3) / 1e9,
         "arith_intensity": 0.0, "stability": 0.98}
    return {"task": "transpose_2d", "chip": chip, "correct": correct, "metrics": m,
            "kernel_timing": k_t, "reference_timing": r_t, "tg_static_mem_bytes": 16640,
            "pso_max_threads_per_tg": 256, "outputs": [{"ok": correct, "max_err": 0.0}],
            "compute_dtype": "f32"}


def test_allclose_semantics():
    ok, err = harness._allclose(np.ones(3), np.ones(4), 0, 0)
    assert (ok, err) == (False, float("inf"))
    assert harness._allclose(np.array([1.0, 2.0]), np.array([1.0, 2.0]), 0, 0) == (True, 0.0)
    assert not harness._allclose(np.array([1.0, np.nan]), np.array([1.0, 2.0]), 1, 1)[0]
    ok, err = harness._allclose(np.array([1.011]), np.array([1.0]), 1e-2, 1e-3)
    assert ok and abs(err - 0.011) < 1e-12
    assert not harness._allclose(np.array([1.0111]), np.array([1.0]), 1e-2, 1e-3)[0]


def test_report_text_parses_with_reference_consumer_regexes():
    buf = io.StringIO()
    with redirect_stdout(buf):
        harness._print_report(_fake_result(), "speed", 1.0)
    out = buf.getvalue()
    for key, rx in RX.items():
        assert rx.search(out), f"{key} line missing:\n{out}"
    assert RX["correct"].search(out).group(1).startswith("✓")
    assert float(RX["kernel"].search(out).group(1)) == 0.128
    assert "roofline    : memory-bound" in out
    # certify's awk reads $3 of the '  kernel  ' line
    kline = next(l for l in out.splitlines() if l.startswith("  kernel  "))
    assert kline.split()[2] == "0.128"


def test_session_update_rules(tmp_path):
    sp = tmp_path / "session.json"
    assert harness.update_session("transpose_2d", _fake_result(False), "speed", 10, sp)[0] is False
    assert not sp.exists()
    ok, why = harness.update_session("transpose_2d", _fake_result(True, 0.2), "speed", 10, sp)
    assert ok and "new best" in why
    rec = json.loads(sp.read_text())["amd-instinct-mi355x"]["transpose_2d"]
    for key in ("best_time_ms", "speedup_vs_mlx", "gflops", "gbps", "arith_intensity", "stability",
                "tg_static_mem_bytes", "pso_max_threads_per_tg", "iters", "target", "max_err",
                "metal_source_path", "metal_source", "updated_at"):
        assert key in rec
    assert rec["metal_source_path"].endswith("transpose.hip")
    assert harness.update_session("transpose_2d", _fake_result(True, 0.3), "speed", 10, sp)[0] is False
    assert harness.update_session("transpose_2d", _fake_result(True, 0.1), "speed", 10, sp)[0] is True
    assert harness._update_best_times_md(sp, tmp_path)
    best = (tmp_path / "best_times.md").read_text()
    row = next(line for line in best.splitlines() if line.startswith("| `transpose_2d` |"))
    cells = [c.strip() for c in row.strip("|").split("|")]
    # reference scripts/render_best_times.py format: kernel | set | chips..., "ms (speedup×)"
    header = next(line for line in best.splitlines() if line.startswith("| kernel | set |"))
    chips = [c.strip() for c in header.strip("|").split("|")][2:]
    assert chips[0] == "amd-instinct-mi355x" and chips[1:] == ["M1", "M2", "M3", "M4", "M5"]
    assert cells[:2] == ["`transpose_2d`", "common"]
    assert cells[2] == f"0.100 ({74.5 / 0.1:.2f}×)" and cells[3:] == ["—"] * 5
    link = (tmp_path / "LINK.md").read_text()
    assert "## amd-instinct-mi355x\n" in link and "## apple-m2 _(no data)_" in link
    # every kernel with data links to the HIP file that registers it
    target = link.split("[transpose_2d](")[1].split(")")[0]
    assert target == "metalbench_amd/csrc/transpose.hip" and (REPO / target).is_file()
    assert "- [llama_decoder_layer](metalbench_amd/csrc/transformer_f32.hip)" in link


def test_grade_targets():
    m = {"speedup": 2.0, "gflops": 1000.0, "gbps": 5.0, "stability": 1.0}
    assert harness.grade(m, "speed") == 2.0
    assert harness.grade(m, "balanced") == pytest.approx(0.5 * 2 + 0.3 * 1 + 0.2 * 1)
    with pytest.raises(SystemExit):
        harness.grade(m, "nope")


def test_roofline_classification_on_mi355x_peaks():
    t = roofline.classify("gfx950", 0, 536870912, 0.0959)
    assert t["classification"] == "memory-bound" and t["sol"] == pytest.approx(0.70, abs=0.01)
    g = roofline.classify("gfx950", 1_099_511_627_776, 402_653_184, 0.7282, "bf16")
    assert g["classification"] == "compute-bound" and g["sol"] == pytest.approx(0.60, abs=0.01)
    d = roofline.classify("gfx950", 7_516_454_912, 570_753_024, 0.07134, "bf16")
    assert d["classification"] == "memory-bound" and d["sol"] == pytest.approx(1.0, abs=0.01)


def test_cli_dry_run_and_cpu_only():
    r = subprocess.run([sys.executable, "mlx/scripts/harness.py", "conv2d", "--dry-run"],
                       cwd=REPO, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    m = json.loads(r.stdout)
    assert m["function"] == "conv2d_f32"
    assert [b["binding"] for b in m["buffers"]][:3] == [0, 1, 2]
    assert {"binding": 11, "role": "scalar", "dtype": "u32", "value": 1} in m["buffers"]
    r = subprocess.run([sys.executable, "mlx/scripts/harness.py", "sqr_mm", "--mlx-only",
                        "--iters", "2"], cwd=REPO, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "mlx ref     :" in r.stdout


def test_profile_counter_parsing_and_absent_profiler(tmp_path, monkeypatch):
    csv_path = tmp_path / "p_counter_collection.csv"
    csv_path.write_text(
        "Dispatch_Id,Kernel_Name,Counter_Name,Counter_Value\n"
        '1,"void mb::(anonymous namespace)::skinny_gemm_kernel<0, 4>(...)",FETCH_SIZE,100.5\n'
        "2,void mb::(anonymous namespace)::attention_kernel<4>(...),FETCH_SIZE,50\n"
        "3,at::native::vectorized_elementwise_kernel,FETCH_SIZE,7\n"
        "2,void mb::(anonymous namespace)::attention_kernel<4>(...),GRBM_GUI_ACTIVE,9\n")
    got = harness.parse_counter_csv(csv_path)
    assert got == {"FETCH_SIZE": 150.5, "GRBM_GUI_ACTIVE": 9.0}   # torch's kernel excluded
    # one pass may hold at most 8 SQ, 4 TCC (FETCH_SIZE 3, WRITE_SIZE 2) and 2 GRBM counters
    for p in harness.PROFILE_PASSES:
        sq = sum(c.startswith("SQ_") for c in p)
        tcc = 3 * ("FETCH_SIZE" in p) + 2 * ("WRITE_SIZE" in p)
        grbm = sum(c.startswith("GRBM_") for c in p)
        assert sq <= 8 and tcc <= 4 and grbm <= 2, p
    import shutil
    monkeypatch.setattr(shutil, "which", lambda name: None)
    prof = harness.profile_counters("sqr_mm", 0)
    assert prof["counters_available"] is False and "rocprofv3" in prof["reason"]


def test_cli_xcode_flags_reach_the_manifest():
    """--xcode / --gputracer / --capture-host parse as in the reference
    (mlx/scripts/harness.py:395-400) and put `capture_path` in the manifest
    (mlx_helpers.py:333-334); --dry-run makes no GPU call."""
    for flag in ("--xcode", "--gputracer"):
        r = subprocess.run([sys.executable, "mlx/scripts/harness.py", "sqr_mm", flag, "--dry-run"],
                           cwd=REPO, capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stderr
        m = json.loads(r.stdout)
        assert m["capture_path"].endswith("/sqr_mm.trace")
        assert "[xcode] will record a kernel trace" in r.stderr
    r = subprocess.run([sys.executable, "mlx/scripts/harness.py", "transpose_2d", "--dry-run",
                        "--capture-host", "/tmp/mb_cap"], cwd=REPO, capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert json.loads(r.stdout)["capture_path"] == "/tmp/mb_cap"
    r = subprocess.run([sys.executable, "mlx/scripts/harness.py", "transpose_2d", "--dry-run"],
                       cwd=REPO, capture_output=True, text=True, timeout=120)
    assert "capture_path" not in json.loads(r.stdout)


def test_kernel_trace_parsing_and_absent_profiler(tmp_path, monkeypatch):
    csv_path = tmp_path / "x_kernel_trace.csv"
    csv_path.write_text(
        '"Kind","Dispatch_Id","Kernel_Name","Start_Timestamp","End_Timestamp"\n'
        '"KERNEL_DISPATCH",3,"mb::(anonymous namespace)::attention_kernel<4>(mb::AttnArgs)",100,2600\n'
        '"KERNEL_DISPATCH",1,"void at::native::vectorized_elementwise_kernel<4>(int)",0,50\n'
        '"KERNEL_DISPATCH",2,"mb::(anonymous namespace)::qkv_kernel(mb::QkvArgs)",60,90\n')
    got = harness.parse_kernel_trace_csv(csv_path)
    assert [k["duration_ns"] for k in got] == [30, 2500]     # dispatch order, torch's excluded
    assert "qkv_kernel" in got[0]["name"]
    import shutil
    monkeypatch.setattr(shutil, "which", lambda name: None)
    cap = harness.capture_dispatch("sqr_mm", 0, tmp_path / "t.trace")
    assert cap["written"] is False and "rocprofv3" in cap["reason"]
    assert harness.available_counter_sets() == []


def test_report_prints_counter_sets_and_trace():
    res = _fake_result()
    res["available_counter_sets"] = ["GRBM_GUI_ACTIVE", "FETCH_SIZE"]
    res["capture"] = {"written": True, "path": "/x/transpose_2d.trace",
                      "kernels": [{"name": "mb::(anonymous namespace)::transpose_kernel(float const*)",
                                   "duration_ns": 93100}]}
    buf = io.StringIO()
    with redirect_stdout(buf):
        harness._print_report(res, "speed", 1.0)
    out = buf.getvalue()
    # the reference prints the counter sets right after the occupancy line (harness.py:295-297)
    lines = out.splitlines()
    i = next(n for n, l in enumerate(lines) if l.startswith("  occupancy   :"))
    assert lines[i + 1] == "  counters    : GRBM_GUI_ACTIVE, FETCH_SIZE"
    assert "  trace       : /x/transpose_2d.trace" in out
    assert re.search(r"transpose_kernel\s+93\.1 µs", out)


def test_bench_script_dispatches_gputracer(tmp_path):
    """`./bench --gputracer <name>` and `./bench <name> --xcode` reach the
    harness with --xcode, and `--gputracer --all` walks every registry set
    (reference bench:17-40).  A stub python3 on PATH records the calls."""
    stub = tmp_path / "python3"
    log = tmp_path / "calls"
    stub.write_text(f"""#!/bin/bash
if [ "$1" = "-c" ]; then exec {sys.executable} "$@"; fi
echo "$*" >> {log}
echo "[host] trace written: /x"
""")
    stub.chmod(0o755)
    import os
    env = dict(os.environ, SKIP_BUILD="1", PATH=f"{tmp_path}:{os.environ['PATH']}")
    for argv in (["--gputracer", "conv2d"], ["conv2d", "--xcode"], ["conv2d", "--gputracer"]):
        log.write_text("")
        r = subprocess.run(["./bench", *argv], cwd=REPO, capture_output=True, text=True,
                           timeout=60, env=env)
        assert r.returncode == 0, r.stderr
        call = log.read_text().split()
        assert call[:2] == ["mlx/scripts/harness.py", "conv2d"] and "--xcode" in call, call
        assert "--save" not in call
    log.write_text("")
    r = subprocess.run(["./bench", "--gputracer", "--all"], cwd=REPO, capture_output=True,
                       text=True, timeout=120, env=env)
    assert r.returncode == 0, r.stderr
    calls = [c.split() for c in log.read_text().splitlines()]
    names = {c[1] for c in calls}
    assert {"sqr_mm", "transpose_2d", "conv2d", "large_mm", "llama_decoder_step"} <= names
    assert all(c[2:4] == ["--xcode", "--metal-only"] for c in calls)
    assert r.stdout.count("trace written") == len(calls)
