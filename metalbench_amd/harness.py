"""MetalBench harness on gfx950: dispatch a kernel, time it, grade it.

    python mlx/scripts/harness.py <name> [--target speed|compute|memory|stable|balanced]
                                         [--iters 200] [--warmup 10] [--seed 0]
                                         [--save] [--no-session] [--dry-run] [--cold-start]
                                         [--profile] [--xcode | --gputracer] [--capture-host DIR]
                                         [--mlx-only | --metal-only] [--cpu-iters N]

Same flow, report text, exit codes and persistence as reference
mlx/scripts/harness.py:52-508, with the gfx950 backend in place of Metal:
  * the kernel runs in-process through libmbhip.so (`mb_run`), on device
    buffers that torch allocates; no manifest/.bin files (reference :36-49, :74-98);
  * the `mlx ref` line times the registry's Model spec on the host CPU
    (MLX does not run on this platform); the correctness gate compares against
    the same spec's output, in float64, with the reference's rule
    |a - b| <= atol + rtol*|b| (reference :26-33);
  * the `roofline` line prices the kernel against MI355X peaks for the dtype
    it computes in;
  * `--profile` and `--capture-host` / `--xcode` run one more dispatch in a
    child process under rocprofv3 (counters, or a kernel trace) instead of
    sampling MTLCounterSet or recording a .gputrace in the host.
`--metal-only` / `--mlx-only` keep their reference meaning: the GPU kernel only
(no spec timing, no correctness gate) / the CPU spec only.
"""
from __future__ import annotations

import argparse
import datetime as _dt
import json
import os
import sys
from pathlib import Path

import numpy as np

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
    from metalbench_amd import helpers as H          # noqa: E402
    from metalbench_amd import native, roofline      # noqa: E402
    from metalbench_amd.timing import time_cpu       # noqa: E402
else:
    from . import helpers as H
    from . import native, roofline
    from .timing import time_cpu


def _to_np64(x) -> np.ndarray:
    if hasattr(x, "detach"):
        x = x.detach().float().cpu().numpy()
    return np.asarray(x).astype(np.float64)


def _allclose(actual, expected, rtol, atol):
    """float64 |a - b| <= atol + rtol*|b| (reference harness.py:26-33)."""
    a = _to_np64(actual)
    b = _to_np64(expected)
    if a.shape != b.shape:
        return False, float("inf")
    if a.size == 0:
        return True, 0.0
    diff = np.abs(a - b)
    tol = atol + rtol * np.abs(b)
    ok = bool(np.all(diff <= tol))     # NaN anywhere fails
    return ok, float(np.nanmax(diff)) if not np.isnan(diff).all() else float("inf")


def _run_native(b, inputs, warmup, iters, flags=native.RUN_SYNC_EACH):
    """Upload inputs, bind, time through mb_run, download outputs.  Replaces
    the host subprocess (reference harness.py:36-49 and main.mm:125-171)."""
    import torch
    native.init(0)
    dev = torch.device("cuda", 0)
    d_in = [t.to(dev) for t in inputs]
    d_out = [torch.zeros(tuple(o.shape), dtype=H.torch_dtype(o.dtype), device=dev)
             for o in b.outputs]
    torch.cuda.synchronize()
    bindings = []
    for binding, t, dt in zip(b.input_bindings, d_in, b.input_dtypes):
        bindings.append(native.make_binding(binding, native.ROLE_INPUT, dt, t.data_ptr(),
                                            t.numel() * t.element_size()))
    for o, t in zip(b.outputs, d_out):
        bindings.append(native.make_binding(o.binding, native.ROLE_OUTPUT, o.dtype,
                                            t.data_ptr(), t.numel() * t.element_size()))
    for s in b.scalars():
        bindings.append(native.make_binding(s.binding, native.ROLE_SCALAR, s.dtype,
                                            value=s.value))
    kid = native.kernel_find(b.metal_function)
    k_t = native.run(kid, bindings, warmup, iters, flags)
    outs = [t.cpu() for t in d_out]
    attrs = native.kernel_attrs(kid)
    k_t["tg_static_mem_bytes"] = attrs["static_lds_bytes"]
    k_t["pso_max_threads_per_tg"] = attrs["max_threads_per_block"]
    k_t["vgprs"] = attrs["num_regs"]
    for key in ("arch_vgprs", "agprs", "sgprs", "waves_per_simd"):
        k_t[key] = attrs[key]
    k_t["hip_device"] = H.chip_info()["name"]
    del d_in, d_out
    return k_t, outs


def _cpu_iters(b, iters, override):
    if override:
        return int(override)
    return max(1, min(int(iters), int(b.meta.get("cpu_iters", iters))))


def evaluate(name, *, seed, warmup, iters, dry_run=False, profile=False, solo=None,
             cpu_iters=None, cold_start=False, capture_host=None):
    b = H.load_baseline(name)
    inputs = b.make_inputs(seed)
    # --mlx-only and --dry-run make no GPU call
    chip = H.host_chip_info() if (solo == "mlx" or dry_run) else H.chip_info()
    c_iters = _cpu_iters(b, iters, cpu_iters)

    if solo == "mlx":
        ref_out = b.reference(*inputs)
        r_t = time_cpu(b.reference, *inputs, warmup=0 if cold_start else 1, iters=c_iters)
        if cold_start:
            r_t["cold_start"] = True
        return {"task": name, "chip": chip, "solo": "mlx",
                "reference_timing": r_t, "correct": True,
                "metrics": {"stability": max(0.0,
                            1.0 - abs(r_t["median_ms"] - r_t["mean_ms"]) / r_t["mean_ms"]
                            if r_t["mean_ms"] > 0 else 0.0)},
                "outputs": []}

    manifest = H.build_manifest(b, inputs, warmup=warmup, iters=iters,
                                chip_type=chip["type"], profile=profile,
                                capture_host=capture_host)
    if dry_run:
        return {"task": name, "dry_run": True, "manifest": manifest}

    # --cold-start: no warmup, and every timed dispatch starts with the caches
    # evicted (the reference clears MLX's caches and drops the warmup, its
    # timing.py:46-48; its host can purge its buffers, timing.mm:236-246)
    if cold_start:
        warmup = 0
    k_t, kernel_outs = _run_native(b, inputs, warmup, iters,
                                   native.RUN_COLD if cold_start else native.RUN_SYNC_EACH)
    if cold_start:
        k_t["cold_start"] = True
    # the reference host records its trace after the timed dispatches
    # (main.mm:173-177), in every mode that runs the kernel
    capture = capture_dispatch(name, seed, capture_host) if capture_host else None

    def _kernel_metrics(m):
        median_s = k_t["median_ms"] / 1000.0
        if median_s > 0:
            if (f := b.flops(inputs)) is not None:
                m["gflops"] = f / median_s / 1e9
            if (nb := b.bytes(inputs)) is not None:
                m["gbps"] = nb / median_s / 1e9
            if f is not None and nb is not None and nb > 0:
                m["arith_intensity"] = f / nb
        mean_ms = k_t["mean_ms"]
        cv = abs(k_t["median_ms"] - mean_ms) / mean_ms if mean_ms > 0 else 0.0
        m["stability"] = max(0.0, 1.0 - cv)
        return m

    if solo == "metal":
        out = {"task": name, "chip": chip, "solo": "metal", "correct": True,
               "metrics": _kernel_metrics({}), "kernel_timing": k_t, "outputs": [],
               "compute_dtype": b.compute_dtype}
        if capture is not None:
            out["capture"] = capture
        return out

    ref_out = b.reference(*inputs)
    ref_outs = list(ref_out) if isinstance(ref_out, (list, tuple)) else [ref_out]
    r_t = time_cpu(b.reference, *inputs, warmup=1 if c_iters > 1 and not cold_start else 0,
                   iters=c_iters)
    r_t["label"] = "cpu spec (torch, %d threads)" % r_t.get("threads", 0)
    if cold_start:
        r_t["cold_start"] = True

    if len(kernel_outs) != len(ref_outs):
        raise RuntimeError(f"{name}: kernel={len(kernel_outs)} outputs, ref={len(ref_outs)}")

    per_output = []
    for k, r in zip(kernel_outs, ref_outs):
        ok, max_err = _allclose(k, r, b.rtol, b.atol)
        per_output.append({"ok": ok, "max_err": max_err})

    correct = all(o["ok"] for o in per_output)
    speedup = (r_t["median_ms"] / k_t["median_ms"]) if k_t["median_ms"] > 0 else float("inf")
    metrics = _kernel_metrics({"speedup": speedup})

    result = {
        "task": name,
        "chip": chip,
        "metal_device": k_t.get("hip_device", "unknown"),
        "tg_static_mem_bytes": k_t.get("tg_static_mem_bytes"),
        "pso_max_threads_per_tg": k_t.get("pso_max_threads_per_tg"),
        "registers": {k: k_t.get(k) for k in ("arch_vgprs", "agprs", "sgprs", "waves_per_simd")},
        "correct": correct,
        "metrics": metrics,
        "speedup": speedup,
        "kernel_timing": k_t,
        "reference_timing": r_t,
        "outputs": per_output,
        "compute_dtype": b.compute_dtype,
    }
    # The reference host always emits the available counter sets and a
    # profiling block (main.mm:181-195); with --profile the block holds
    # counters, here from rocprofv3 passes.
    result["available_counter_sets"] = available_counter_sets()
    result["profiling"] = profile_counters(name, seed) if profile else {"counters_available": False}
    if capture is not None:
        result["capture"] = capture
    return result


# ---- --profile: hardware counters through rocprofv3 --------------------------------------
# The reference samples MTLCounterSet around one extra dispatch (reference
# harness.py:401-402, main.mm:53-72).  Here the same registry kernel is run
# once more in a child process under `rocprofv3 --pmc`, one pass per counter
# group (a pass may hold at most 8 SQ, 4 TCC and 2 GRBM counters; FETCH_SIZE
# takes 3 TCC and WRITE_SIZE 2, so they go in separate passes), and the values
# are summed over the kernels of that one dispatch.
PROFILE_PASSES = (
    ("GRBM_GUI_ACTIVE", "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES", "SQ_INSTS_MFMA",
     "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE",
     "SQ_WAIT_INST_LDS", "SQ_WAIT_INST_ANY", "FETCH_SIZE"),
    ("WRITE_SIZE",),
)


def available_counter_sets() -> list:
    """What `--profile` can sample on this host: the counters of its
    rocprofv3 passes, or nothing without rocprofv3 (the reference lists the
    device's MTLCounterSets, main.mm:40-51)."""
    import shutil
    if not shutil.which("rocprofv3"):
        return []
    return [c for p in PROFILE_PASSES for c in p]


def parse_counter_csv(path) -> dict:
    """Sum each counter over this library's kernels in a rocprofv3
    counter_collection.csv."""
    import csv
    out = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if "mb::" not in r.get("Kernel_Name", ""):
                continue
            out[r["Counter_Name"]] = out.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return out


def profile_counters(name, seed, timeout_s=120) -> dict:
    import shutil
    import subprocess
    import tempfile
    exe = shutil.which("rocprofv3")
    if not exe:
        return {"counters_available": False, "reason": "rocprofv3 not found"}
    env = dict(os.environ, TMPDIR="/tmp")
    values = {}
    for counters in PROFILE_PASSES:
        with tempfile.TemporaryDirectory(dir="/tmp") as d:
            cmd = [exe, "--pmc", *counters, "-f", "csv", "-d", d, "-o", "prof", "--",
                   sys.executable, str(H.REPO_ROOT / "mlx" / "scripts" / "harness.py"), name,
                   "--metal-only", "--warmup", "0", "--iters", "1", "--seed", str(seed),
                   "--no-session"]
            try:
                r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout_s,
                                   cwd="/tmp", env=env)
            except subprocess.TimeoutExpired:
                return {"counters_available": False, "reason": f"rocprofv3 pass timed out ({counters[0]} ...)"}
            found = list(Path(d).rglob("*counter_collection.csv"))
            if r.returncode != 0 or not found:
                return {"counters_available": False,
                        "reason": f"rocprofv3 exit {r.returncode}: {r.stderr.strip()[-200:]}"}
            values.update(parse_counter_csv(found[0]))
    names = [c for p in PROFILE_PASSES for c in p]
    return {"counters_available": True, "counter_set": "rocprofv3 --pmc (" + ", ".join(names) + ")",
            "samples": [{"name": c, "value": int(values.get(c, 0))} for c in names]}


# ---- --capture-host / --xcode: a kernel trace of one dispatch --------------------------
# The reference records a .gputrace of one extra dispatch (timing.mm:199-229,
# reached through the manifest's capture_path, main.mm:173-177).  Here the
# registry kernel runs once more in a child process under
# `rocprofv3 --kernel-trace --stats`, which writes its CSV files into the
# capture directory; the report names the kernels of that dispatch.
def parse_kernel_trace_csv(path) -> list:
    """This library's kernels in a rocprofv3 kernel_trace.csv, in dispatch
    order: [{"name", "duration_ns"}]."""
    import csv
    rows = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if "mb::" not in r.get("Kernel_Name", ""):
                continue
            rows.append((int(r.get("Dispatch_Id") or 0), r["Kernel_Name"],
                         int(r["End_Timestamp"]) - int(r["Start_Timestamp"])))
    rows.sort()
    return [{"name": n, "duration_ns": d} for _, n, d in rows]


def capture_dispatch(name, seed, trace_path, timeout_s=180) -> dict:
    import shutil
    import subprocess
    out = Path(trace_path).resolve()
    exe = shutil.which("rocprofv3")
    if not exe:
        print("[host] capture unavailable: rocprofv3 not found", file=sys.stderr)
        return {"written": False, "path": str(out), "reason": "rocprofv3 not found"}
    out.mkdir(parents=True, exist_ok=True)
    env = dict(os.environ, TMPDIR="/tmp")
    cmd = [exe, "--kernel-trace", "--stats", "-f", "csv", "-d", str(out), "-o", name, "--",
           sys.executable, str(H.REPO_ROOT / "mlx" / "scripts" / "harness.py"), name,
           "--metal-only", "--warmup", "0", "--iters", "1", "--seed", str(seed),
           "--no-session"]
    try:
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout_s,
                           cwd="/tmp", env=env)
    except subprocess.TimeoutExpired:
        print(f"[host] capture unavailable: rocprofv3 timed out after {timeout_s} s",
              file=sys.stderr)
        return {"written": False, "path": str(out), "reason": "rocprofv3 timed out"}
    found = sorted(out.rglob(f"{name}_kernel_trace.csv"))
    if r.returncode != 0 or not found:
        why = f"rocprofv3 exit {r.returncode}: {r.stderr.strip()[-200:]}"
        print(f"[host] capture unavailable: {why}", file=sys.stderr)
        return {"written": False, "path": str(out), "reason": why}
    kernels = parse_kernel_trace_csv(found[-1])
    print(f"[host] trace written: {out}", file=sys.stderr)
    return {"written": True, "path": str(out), "files": [str(p) for p in sorted(out.rglob("*.csv"))],
            "kernels": kernels}


# Each target picks ONE primary metric to optimize (reference harness.py:176-186).
TARGETS = {
    "speed": lambda m: m.get("speedup", 0.0),
    "compute": lambda m: m.get("gflops", 0.0),
    "memory": lambda m: m.get("gbps", 0.0),
    "stable": lambda m: m.get("stability", 0.0),
    "balanced": lambda m: (
        0.5 * m.get("speedup", 0.0)
        + 0.3 * (m.get("gflops", 0.0) / 1000.0)
        + 0.2 * m.get("stability", 0.0)
    ),
}


def grade(metrics, target):
    fn = TARGETS.get(target)
    if fn is None:
        raise SystemExit(f"unknown target '{target}'; pick {list(TARGETS)}")
    return float(fn(metrics))


def update_session(name, result, target, iters, session_path=None):
    """Best run per (chip bucket, kernel) in session.json, same keys as
    reference harness.py:196-247: updated only if correct and faster.  The
    kernel source stored is the HIP file that implements the kernel."""
    if not result.get("correct"):
        return False, "skipped (incorrect)"
    session_path = Path(session_path) if session_path else H.SESSION_PATH
    bucket = result["chip"]["bucket"]
    new_ms = result["kernel_timing"]["median_ms"]

    src_path = H.find_kernel_source(name)
    src_text = src_path.read_text() if src_path else None

    session = {}
    if session_path.exists():
        try:
            session = json.loads(session_path.read_text())
        except Exception:
            session = {}

    chip_section = session.setdefault(bucket, {})
    prev = chip_section.get(name)
    prev_ms = prev["best_time_ms"] if prev else None
    if prev_ms is not None and new_ms >= prev_ms:
        return False, f"current best {prev_ms:.3f} ms holds (this run {new_ms:.3f} ms)"

    try:
        rel_src = str(src_path.relative_to(H.REPO_ROOT)) if src_path else None
    except ValueError:
        rel_src = str(src_path)
    chip_section[name] = {
        "best_time_ms": new_ms,
        "speedup_vs_mlx": result["metrics"]["speedup"],
        "gflops": result["metrics"].get("gflops"),
        "gbps": result["metrics"].get("gbps"),
        "arith_intensity": result["metrics"].get("arith_intensity"),
        "stability": result["metrics"]["stability"],
        "tg_static_mem_bytes": result.get("tg_static_mem_bytes"),
        "pso_max_threads_per_tg": result.get("pso_max_threads_per_tg"),
        "iters": iters,
        "target": target,
        "max_err": max((o["max_err"] for o in result["outputs"]), default=0.0),
        "metal_source_path": rel_src,
        "metal_source": src_text,
        "updated_at": _dt.datetime.now(_dt.timezone.utc).isoformat(timespec="seconds"),
    }
    session_path.write_text(json.dumps(session, indent=2) + "\n")
    delta = "" if prev_ms is None else f" (was {prev_ms:.3f} ms, Δ {prev_ms - new_ms:+.3f})"
    return True, f"new best {new_ms:.3f} ms{delta}"


def _bytes_human(n):
    for u in ("B", "KB", "MB", "GB"):
        if n < 1024:
            return f"{n:.0f}{u}"
        n /= 1024
    return f"{n:.0f}TB"


def _roofline_line(result, m, k_t):
    f = m.get("gflops", 0) * (k_t["median_ms"] / 1000.0) * 1e9 if "gflops" in m else 0
    nb = m.get("gbps", 0) * (k_t["median_ms"] / 1000.0) * 1e9 if "gbps" in m else 0
    rl = roofline.classify(result["chip"]["type"], f, nb, k_t["median_ms"],
                           result.get("compute_dtype", "f32"))
    return roofline.format_line(rl)


def _print_capture(cap):
    if not cap:
        return
    if not cap.get("written"):
        print(f"  trace       : unavailable ({cap.get('reason')})")
        return
    print(f"  trace       : {cap['path']}  (rocprofv3 kernel trace of one dispatch)")
    for k in cap.get("kernels", []):
        short = k["name"].replace("(anonymous namespace)::", "").split("(")[0]
        print(f"    {short:40s} {k['duration_ns'] / 1000.0:10.1f} µs")


def _print_report(result, target, score):
    """Human-readable report, same labels as reference harness.py:257-333."""
    chip = result["chip"]
    m = result["metrics"]
    k_t = result.get("kernel_timing")
    r_t = result.get("reference_timing")
    outs = result.get("outputs", [])
    solo = result.get("solo")

    line = "─" * 72
    if solo:
        side = "MLX only" if solo == "mlx" else "Metal only"
        print(line); print(f"  {result['task']}    [{side}]"); print(line)
        print(f"  device      : {chip['name']} ({chip['type']})  "
              f"{chip['cpu_cores']} CPU / {chip['gpu_cores']} GPU / "
              f"{chip['ram_bytes']/1e9:.0f} GB")
        t = k_t if solo == "metal" else r_t
        label = "metal kernel" if solo == "metal" else "mlx ref"
        print(f"  {label:11s} : {t['median_ms']:.3f} ms  "
              f"(min {t['min_ms']:.3f}, mean {t['mean_ms']:.3f}, n={t['iters']})")
        if "gflops" in m: print(f"  compute     : {m['gflops']:.1f} GFLOPS")
        if "gbps" in m: print(f"  bandwidth   : {m['gbps']:.1f} GB/s")
        if "stability" in m:
            print(f"  stability   : {m['stability']:.2f}")
        if solo == "metal":
            print(_roofline_line(result, m, k_t))
            _print_capture(result.get("capture"))
        print(line)
        return

    print(line)
    print(f"  {result['task']}    target={target}   score={score:.3f}")
    print(line)
    print(f"  device      : {chip['name']} ({chip['type']})  "
          f"{chip['cpu_cores']} CPU / {chip['gpu_cores']} GPU / "
          f"{chip['ram_bytes']/1e9:.0f} GB")
    if result.get("tg_static_mem_bytes") is not None:
        regs = result.get("registers") or {}
        extra = ""
        if (regs.get("arch_vgprs") or -1) >= 0:
            extra = (f"  vgpr={regs['arch_vgprs']} agpr={regs['agprs']} sgpr={regs['sgprs']}"
                     f"  waves/simd={regs['waves_per_simd']}")
        print(f"  occupancy   : tg_mem={_bytes_human(result['tg_static_mem_bytes'])}  "
              f"max_thr/tg={result['pso_max_threads_per_tg']}{extra}")
    if result.get("available_counter_sets"):
        print(f"  counters    : {', '.join(result['available_counter_sets'])}")
    print()
    status = "✓ correct " if result["correct"] else "✗ INCORRECT"
    max_err = max((o["max_err"] for o in outs), default=0.0)
    print(f"  correctness : {status}    max_err={max_err:.3e}")
    print(f"  speedup     : {m.get('speedup', 0):.2f}× vs MLX")
    print(f"  kernel      : {k_t['median_ms']:.3f} ms  "
          f"(min {k_t['min_ms']:.3f}, mean {k_t['mean_ms']:.3f}, n={k_t['iters']})")
    print(f"  mlx ref     : {r_t['median_ms']:.3f} ms  "
          f"(min {r_t['min_ms']:.3f}, mean {r_t['mean_ms']:.3f}, n={r_t['iters']})"
          f"  [{r_t.get('label', 'cpu spec')}]")
    if "gflops" in m:
        print(f"  compute     : {m['gflops']:.1f} GFLOPS")
    if "gbps" in m:
        print(f"  bandwidth   : {m['gbps']:.1f} GB/s")
    if "arith_intensity" in m:
        print(f"  arith int.  : {m['arith_intensity']:.1f} FLOPs/byte")
    print(f"  stability   : {m['stability']:.2f}  (1.0 = perfectly consistent)")
    try:
        print(_roofline_line(result, m, k_t))
    except Exception:
        pass
    for p in k_t.get("parts", []):
        print(f"    part {p['name']:24s} {p['median_ms']*1000:8.1f} µs")
    prof = result.get("profiling", {})
    if prof.get("counters_available"):
        print(f"  profiling   : {prof['counter_set']}")
        for smp in prof.get("samples", []):
            print(f"    {smp['name']:40s} {smp['value']}")
    elif prof.get("reason"):
        print(f"  profiling   : unavailable ({prof['reason']})")
    _print_capture(result.get("capture"))
    print()
    print(f"  {'target':>10s}   {'score':>10s}")
    print(f"  {'-'*10}   {'-'*10}")
    for t in ("speed", "compute", "memory", "stable", "balanced"):
        s = grade(m, t)
        print(f"  {t:>10s}   {s:10.3f}")
    print(line)


def _update_best_times_md(session_path=None, out_dir=None):
    """Regenerate best_times.md and LINK.md from session.json (reference
    harness.py:336-384, scripts/render_best_times.py, scripts/render_link_md.py)."""
    from . import render
    return render.update_markdown(session_path, out_dir)


def main(argv=None):
    ap = argparse.ArgumentParser(prog="metalbench-harness")
    ap.add_argument("name", nargs="?")
    ap.add_argument("--_update_md", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--iters", type=int, default=200)
    ap.add_argument("--cpu-iters", type=int, default=None,
                    help="iterations of the CPU spec timing (default: registry cpu_iters)")
    ap.add_argument("--dry-run", action="store_true")
    ap.add_argument("--cold-start", action="store_true",
                    help="no warmup; evict every cache level before each timed dispatch")
    ap.add_argument("--profile", action="store_true",
                    help="hardware counters of one extra dispatch, from rocprofv3 --pmc passes")
    ap.add_argument("--capture-host", default=None, metavar="DIR",
                    help="rocprofv3 kernel trace of one extra dispatch, written into DIR")
    ap.add_argument("--xcode", "--gputracer", dest="xcode", action="store_true",
                    help="kernel trace of one extra dispatch into results/<chip>/<name>.trace "
                         "(--gputracer is an alias)")
    ap.add_argument("--save", action="store_true",
                    help="save full result JSON to results/<chip>/<name>.json")
    ap.add_argument("--no-session", action="store_true", help="don't update session.json")
    ap.add_argument("--target", default="speed", choices=list(TARGETS.keys()))
    solo = ap.add_mutually_exclusive_group()
    solo.add_argument("--mlx-only", action="store_true",
                      help="time only the CPU spec (no GPU call)")
    solo.add_argument("--metal-only", action="store_true",
                      help="time only the gfx950 kernel (skip spec timing + correctness)")
    args = ap.parse_args(argv)
    solo_mode = "mlx" if args.mlx_only else ("metal" if args.metal_only else None)

    if args._update_md:
        _update_best_times_md()
        return 0
    if not args.name:
        ap.error("kernel name required (or use --all from bench script)")

    gpu_call = solo_mode != "mlx" and not args.dry_run
    chip = H.chip_info() if gpu_call else H.host_chip_info()
    if gpu_call and chip["type"] != "gfx950":
        sys.exit(f"[error] this backend requires an AMD gfx950 (MI355X) GPU. "
                 f"Detected: {chip.get('error', chip['name'])!r}.")

    print(f"[chip] {chip['type']:>8s}  '{chip['name']}'  "
          f"cpu={chip['cpu_cores']}  gpu={chip['gpu_cores']}  "
          f"ram={chip['ram_bytes']/1e9:.0f}GB", file=sys.stderr)

    try:
        bf = H.load_baseline(args.name).best_for
        if bf and "all" not in bf and chip["type"] not in bf:
            print(f"[bench] kernel `{args.name}` BEST_FOR={list(bf)}; "
                  f"current chip '{chip['type']}' not in that list", file=sys.stderr)
        elif bf:
            print(f"[bench] kernel `{args.name}` BEST_FOR={list(bf)}", file=sys.stderr)
    except Exception:
        pass

    # --xcode: the trace goes to results/<chip type>/<name>.trace unless
    # --capture-host names a place (reference harness.py:455-464); there is no
    # viewer to open, so the report prints its kernels instead
    if args.xcode and args.capture_host is None:
        args.capture_host = str(H.RESULTS_ROOT / chip["type"] / f"{args.name}.trace")
        print(f"[xcode] will record a kernel trace → {args.capture_host}", file=sys.stderr)
    if args.capture_host and solo_mode == "mlx":
        print("[xcode] no trace: --mlx-only makes no GPU call", file=sys.stderr)

    result = evaluate(args.name, seed=args.seed, warmup=args.warmup, iters=args.iters,
                      dry_run=args.dry_run, profile=args.profile, solo=solo_mode,
                      cpu_iters=args.cpu_iters, cold_start=args.cold_start,
                      capture_host=args.capture_host)

    if args.dry_run:
        print(json.dumps(result["manifest"], indent=2))
        return 0

    score = grade(result["metrics"], args.target)
    result["target"] = args.target
    result["score"] = score
    _print_report(result, args.target, score)

    if solo_mode:
        return 0

    if args.save:
        out_dir = H.RESULTS_ROOT / result["chip"]["bucket"]
        out_dir.mkdir(parents=True, exist_ok=True)
        out_path = out_dir / f"{args.name}.json"
        out_path.write_text(json.dumps(result, indent=2, default=str))
        print(f"saved → {out_path.relative_to(H.REPO_ROOT)}", file=sys.stderr)

    if not args.no_session:
        updated, why = update_session(args.name, result, args.target, args.iters)
        rel = H.SESSION_PATH.relative_to(H.REPO_ROOT)
        prefix = f"updated {rel}" if updated else f"{rel} unchanged"
        print(f"{prefix} [{result['chip']['bucket']}/{args.name}]: {why}", file=sys.stderr)

    return 0 if result["correct"] else 1


if __name__ == "__main__":
    sys.exit(main())
