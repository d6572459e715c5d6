#!/usr/bin/env python3
"""Driver benchmark: one JSON line for the kernel-registry hot path on MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

A "step" is one dispatch of a registry entry over one batch of synthetic,
seeded input already resident in HBM.  The headline workload is the LLaMA
decoder decode step ("decoder block us/step"); the other four
configurations (sqr_mm, transpose_2d, conv2d, large_mm) are timed the same way
and reported under "kernels", each with its own roofline fraction.

Timing: first the workload's own launches keep the GPU busy for --settle-ms
(100 ms; an idle MI355X needs ~30 ms of MFMA work to reach its working
clock), then W untimed steps, then exactly K steps launched back to back with no
events in the stream, bracketed by torch.cuda.synchronize() on both sides;
ms_per_step is the host wall clock of the K steps / K.  The HBM-bound
workloads (decoder step, transpose) are timed cold: each step uses the next of
R device copies of its working set (R x 570 MB for the decoder, R x 536 MB for
the transpose), through the typed C entry point, so the 256 MB memory-side
cache cannot serve one step from the previous one; the others reuse one set
of buffers through mb_run.  Then K more
steps run with a hipEvent pair per step (and, for the decode step, each
kernel's own start and end events, which give `parts`): `roofline.achieved` is the algorithmic bytes (HBM-bound
kernels) or flops (MFMA-bound kernels) of ONE launch of the dominant kernel
divided by that kernel's mean event-timed duration over those K steps.

HBM-bound records also carry `measured_peak` / `frac_of_measured`: the same
achieved rate against what the library's copy kernel moves on this box, cold
(`hbm_measured_gbps`, measured at start-up), beside the datasheet fraction.

cpu_baseline: the registry's torch-CPU Model spec (the harness's `mlx ref`
line) timed on all host cores over the full workload -- a reported baseline,
not a target.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

METRIC = "TFLOP/s or GB/s as % of MI355X roofline per kernel; decoder block µs/step"
HBM_PEAK_GBPS = 8000.0
MFMA_PEAK_TFLOPS = {"f32": 157.3, "bf16": 2516.6}

# Decode-step workloads (registry mlx/kernels/full/registry.py): the whole
# layer and one GPU's share of it under 8-way tensor parallelism.
DECODE_STEPS = ("llama_decoder_step", "llama_decoder_step_tp8")


def _step_shape(meta: dict) -> dict:
    """B, D, H, Hkv, Dh, FF, L of a decode-step registry entry, from its scalars."""
    sc = {s["binding"]: s["value"] for s in meta["scalars"]}
    return dict(B=sc[10], D=sc[11], H=sc[12], HKV=sc[13], DH=128, FF=sc[14], L=sc[15])


def _decoder_part_bytes(meta: dict | None = None) -> dict:
    """Bytes one launch of each decoder kernel must move, for the per-kernel
    `hbm_frac` of `parts`: every weight and cache byte once, plus the kernel's
    own activation inputs and outputs once at the width they are stored in
    (bf16 = 2 bytes; the x1 residual is fp32 and written by W_o, read by
    down).  The QKV GEMM's result reaches attention as split-K partials, which
    neither side counts.  The step's headline roofline does not use these: it
    is priced on the registry's algorithmic bytes (weights, caches, x, y, the
    new k and v), which leave every intermediate out.  The attention width
    QD = H * Dh is D for a whole layer."""
    if meta is None:
        from metalbench_amd import helpers as H
        meta = H.load_baseline("llama_decoder_step").meta
    t = _step_shape(meta)
    B, D, HKV, DH, FF, L = t["B"], t["D"], t["HKV"], t["DH"], t["FF"], t["L"]
    QD = t["H"] * DH
    qkv_n = QD + 2 * HKV * DH
    return {
        "qkv": 2 * (D * qkv_n + B * D),
        "attention": 2 * (2 * B * HKV * L * DH + 2 * B * HKV * DH + B * QD),
        "wo_residual": 2 * (QD * D + B * QD + B * D) + 4 * B * D,
        "gate_up_swiglu": 2 * (D * 2 * FF + B * D + B * FF),
        "down_residual": 2 * (FF * D + B * FF + B * D) + 4 * B * D,
    }


# Per workload: (dominant part name or None for single-kernel, bound, units of
# algorithmic work per launch, unit of `value`).
def _work(name: str, meta: dict):
    if name in DECODE_STEPS:
        # The roofline is priced on the whole step (its five kernels and the
        # dispatch gaps between them) over the back-to-back timed region, with
        # the registry's algorithmic bytes; the per-kernel figures stay in
        # `parts`.
        return dict(part=None, bound="hbm", per_launch=int(meta["bytes"]),
                    parts=_decoder_part_bytes(meta),
                    label="decode step: qkv, attention, wo_residual, gate_up_swiglu, "
                          "down_residual")
    if _bound(meta) == "hbm":
        return dict(part=None, bound="hbm", per_launch=int(meta["bytes"]))
    return dict(part=None, bound="mfma", per_launch=int(meta["flops"]))


def _bound(meta: dict) -> str:
    """HBM if the registry's arithmetic intensity is below the MI355X ridge
    point for its compute dtype (peak flops / 8 TB/s), else MFMA."""
    flops, nbytes = meta.get("flops", 0), meta.get("bytes", 1)
    ridge = MFMA_PEAK_TFLOPS[meta.get("compute_dtype", "f32")] * 1e12 / (HBM_PEAK_GBPS * 1e9)
    return "hbm" if flops / nbytes < ridge else "mfma"


def _value_unit(name: str, meta: dict, ms_per_step: float):
    if name in DECODE_STEPS:
        return ms_per_step * 1000.0, "us/step", False
    if _bound(meta) == "hbm":
        return meta["bytes"] / (ms_per_step * 1e-3) / 1e9, "GB/s", True
    return meta["flops"] / (ms_per_step * 1e-3) / 1e12, "TFLOP/s", True


def _roofline(name: str, w: dict, k_t: dict, compute_dtype: str) -> dict:
    if w["part"] is not None:
        part = next(p for p in k_t.get("parts", []) if p["name"] == w["part"])
        mean_ms = part["mean_ms"]
        kernel = w["part"]
    else:
        # single-kernel workload: average launch duration over the timed region
        mean_ms = k_t.get("device_ms_per_launch", k_t["mean_ms"])
        kernel = None
    sec = mean_ms * 1e-3
    if w["bound"] == "hbm":
        achieved = w["per_launch"] / sec / 1e9
        peak, unit = HBM_PEAK_GBPS, "GB/s"
    else:
        achieved = w["per_launch"] / sec / 1e12
        peak, unit = MFMA_PEAK_TFLOPS[compute_dtype], "TFLOP/s"
    out = {"bound": w["bound"], "achieved": achieved, "peak": peak, "unit": unit,
           "frac": achieved / peak, "traffic": _traffic(kernel or name),
           "kernel_mean_us": mean_ms * 1e3}
    if w["bound"] == "hbm" and "gbps" in _MEASURED_HBM:
        # against what a plain copy kernel moves on this box, cold
        out["measured_peak"] = _MEASURED_HBM["gbps"]
        out["frac_of_measured"] = achieved / _MEASURED_HBM["gbps"]
    if kernel or w.get("label"):
        out["kernel"] = kernel or w["label"]
    return out


def _traffic(key: str) -> float | None:
    """Bytes per launch that left the L2s (FETCH_SIZE x read scale + WRITE_SIZE
    x write scale, both scales from a 256 MiB copy kernel) as recorded from
    rocprofv3 --pmc runs in profiles/traffic.json, keyed by decoder part or
    workload name; None if no counter run has been recorded for it."""
    p = REPO / "profiles" / "traffic.json"
    if not p.is_file():
        return None
    try:
        return json.loads(p.read_text()).get(key, {}).get("bytes_per_launch")
    except Exception:
        return None


def _cpu_baseline(name: str, b, inputs, meta: dict) -> dict:
    """Time the registry's torch-CPU Model spec -- the same callable the
    harness's `mlx ref` line times and the correctness gate compares against --
    on the full workload, on every host core, with the statistics of reference
    mlx/scripts/timing.py:31-72 (untimed warmup, then the median of the sorted
    times), over about 10 s of CPU work.  The spec computes at the
    workload's precision: fp32 for the fp32 entries, the bf16 product with fp32
    accumulation for large_mm, fp32 math on the bf16 weights and cache for the
    decoder step (as the kernels do)."""
    import platform

    import torch

    from metalbench_amd import helpers as H
    from metalbench_amd.timing import time_cpu, use_all_cores

    use_all_cores()
    t0 = time.perf_counter()
    b.reference(*inputs)                     # warmup, and the size of one call
    once = time.perf_counter() - t0
    # ~10 s of timed CPU work (at least 3 calls, at most 500): the 1024^3
    # GEMM's 1.6 ms calls take 500, the 8192^3 bf16 GEMM's ~150 ms calls ~66
    iters = max(3, min(500, int(10.0 / max(once, 1e-6))))
    t = time_cpu(b.reference, *inputs, warmup=0, iters=iters)
    value, unit, _ = _value_unit(name, meta, t["median_ms"])
    return {"value": value, "unit": unit, "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"full workload through the registry's torch-CPU Model spec "
                      f"(torch {torch.__version__}, {torch.get_num_threads()} threads on "
                      f"{H.cpu_model()}, {platform.machine()}); median of {iters} calls "
                      f"({iters * t['mean_ms'] / 1000:.1f} s) after 1 warmup, "
                      f"{t['median_ms']:.1f} ms per step"}


_MEASURED_HBM = {}


def _measured_hbm_gbps() -> float:
    """Achievable HBM bandwidth of this box: the library's copy kernel over
    512 MiB (read) + 512 MiB (write), rotated over two buffer pairs so no
    launch finds its bytes in the 256 MB memory-side cache, after the same
    clock settle as the workloads; device time of 20 back-to-back launches.
    Measured once per process."""
    if "gbps" in _MEASURED_HBM:
        return _MEASURED_HBM["gbps"]
    import ctypes

    import torch

    from metalbench_amd import native

    lib = native.load()
    n = (512 << 20) // 4
    pairs = [(torch.empty(n, device="cuda"), torch.empty(n, device="cuda")) for _ in range(2)]
    for src, _ in pairs:
        src.fill_(1.0)
    stream = torch.cuda.Stream()
    sp = ctypes.c_void_p(stream.cuda_stream)

    def launch_n(count):
        for i in range(count):
            src, dst = pairs[i % 2]
            native.check("mb_launch_copy_f32", lib.mb_launch_copy_f32(src.data_ptr(), dst.data_ptr(),
                                                                       n, sp))
    with torch.cuda.stream(stream):
        _settle(launch_n, 30.0)
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record(stream)
        launch_n(20)
        ev1.record(stream)
    torch.cuda.synchronize()
    sec = ev0.elapsed_time(ev1) / 20 * 1e-3
    _MEASURED_HBM["gbps"] = 2 * n * 4 / sec / 1e9
    del pairs
    return _MEASURED_HBM["gbps"]


def _copy_calibration(n_bytes: int = 256 << 20, launches: int = 3) -> None:
    """Launch the plain (cached) copy kernel over a buffer of known size.
    Under `rocprofv3 --pmc FETCH_SIZE` / `WRITE_SIZE` its counter values are
    the scale that turns the other kernels' counters into bytes."""
    import torch

    from metalbench_amd import native

    n = n_bytes // 4
    src = torch.randn(n, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    b = [native.make_binding(0, native.ROLE_INPUT, "f32", src.data_ptr(), n_bytes),
         native.make_binding(1, native.ROLE_OUTPUT, "f32", dst.data_ptr(), n_bytes),
         native.make_binding(2, native.ROLE_SCALAR, "u32", value=n)]
    native.run(native.kernel_find("copy_f32_plain"), b, 0, launches, native.RUN_PIPELINED)
    torch.cuda.synchronize()
    print(f"[bench] copy calibration: {launches} x copy_f32_plain of {n_bytes} bytes",
          file=sys.stderr, flush=True)


# HBM-bound workloads are timed cold: their working set (weights + KV cache,
# or the matrix being transposed) is rotated over R device copies, so no step
# finds the previous step's bytes in the 256 MB memory-side cache (MALL) -- as
# in a real decode, where every layer streams its own weights and cache.
# The tensor-parallel shard's working set is ~72 MB, so it takes 6 copies
# (5 x 72 MB touched between two uses of one copy > 256 MB).
ROTATE = {"llama_decoder_step": 3, "llama_decoder_step_tp8": 6, "transpose_2d": 2}


def _async_launcher(name, b, copies_in, copies_out):
    """Per-copy launch through the typed C entry point (asynchronous, library
    stream), for the rotating timed loop; None for non-rotating workloads."""
    import ctypes

    from metalbench_amd import native

    lib = native.load()
    sc = {s.binding: s.value for s in b.scalars()}
    if name in DECODE_STEPS:
        args = []
        for ci, co in zip(copies_in, copies_out):
            a = native.MbDecoderStepArgs()
            a.batch, a.d_model, a.n_heads, a.n_kv_heads = sc[10], sc[11], sc[12], sc[13]
            a.head_dim, a.d_ff, a.cache_len, a.cache_stride = 128, sc[14], sc[15], sc[15]
            a.rope_base, a.eps = sc[16], sc[17]
            (a.x, a.w_qkv, a.w_o, a.w_gu, a.w_down, a.k_cache, a.v_cache) = [t.data_ptr() for t in ci]
            a.y, a.k_new, a.v_new = [t.data_ptr() for t in co]
            a.workspace, a.workspace_bytes = None, 0
            args.append(a)

        def launch(c):
            native.check("mb_launch_llama_decoder_step_bf16",
                         lib.mb_launch_llama_decoder_step_bf16(ctypes.byref(args[c]), None))
        return launch
    if name == "transpose_2d":
        rows, cols = sc[2], sc[3]

        def launch(c):
            native.check("mb_launch_transpose_2d_f32", lib.mb_launch_transpose_2d_f32(
                copies_in[c][0].data_ptr(), copies_out[c][0].data_ptr(), rows, cols, None))
        return launch
    return None


def _settle(launch_n, ms: float) -> float:
    """Keep the GPU busy with the workload's own launches for `ms` of wall time
    (batches of launch_n(count), doubled until one takes >= 5 ms, each followed
    by a synchronize); returns the time spent.

    An idle MI355X reaches its working clock only after ~25-30 ms of
    continuous MFMA work: right after an idle second, conv2d launches went
    150 -> 101 -> 93 -> 88 -> 85 -> 83 us over the first 30 ms and the 8192^3
    bf16 GEMM 1306 -> 964 -> 892 -> 832 -> 823 us, flat after that; the
    HBM-bound decode step was flat from its second millisecond.  W warmup
    launches of a 21 us kernel end long before that, so without this the K
    timed steps would measure the ramp."""
    import torch

    t0 = time.perf_counter()
    batch = 1
    while True:
        t1 = time.perf_counter()
        launch_n(batch)
        torch.cuda.synchronize()
        now = time.perf_counter()
        if (now - t0) * 1e3 >= ms:
            return (now - t0) * 1e3
        if (now - t1) * 1e3 < 5.0:
            batch *= 2


def _mean_timing(runs: list) -> dict:
    """Average single-iteration mb_run timings (and their per-kernel parts)."""
    out = {"mean_ms": sum(r["mean_ms"] for r in runs) / len(runs)}
    ms = sorted(r["mean_ms"] for r in runs)
    out["median_ms"] = ms[len(ms) // 2]
    if runs[0].get("parts"):
        out["parts"] = [{"name": p["name"],
                         "mean_ms": sum(r["parts"][i]["mean_ms"] for r in runs) / len(runs)}
                        for i, p in enumerate(runs[0]["parts"])]
    return out


def _run_workload(name, steps, warmup, want_cpu, settle_ms):
    import ctypes

    import torch

    from metalbench_amd import helpers as H
    from metalbench_amd import native

    b = H.load_baseline(name)
    meta = b.meta
    inputs = b.make_inputs(0)
    dev = torch.device("cuda", 0)
    R = ROTATE.get(name, 1)
    copies_in = [[t.to(dev) for t in inputs]]
    copies_out = [[torch.zeros(tuple(o.shape), dtype=H.torch_dtype(o.dtype), device=dev)
                   for o in b.outputs]]
    for _ in range(R - 1):
        copies_in.append([t.clone() for t in copies_in[0]])
        copies_out.append([t.clone() for t in copies_out[0]])

    def bindings_for(ci, co):
        bs = []
        for binding, t, dt in zip(b.input_bindings, ci, b.input_dtypes):
            bs.append(native.make_binding(binding, native.ROLE_INPUT, dt, t.data_ptr(),
                                          t.numel() * t.element_size()))
        for o, t in zip(b.outputs, co):
            bs.append(native.make_binding(o.binding, native.ROLE_OUTPUT, o.dtype, t.data_ptr(),
                                          t.numel() * t.element_size()))
        for s in b.scalars():
            bs.append(native.make_binding(s.binding, native.ROLE_SCALAR, s.dtype, value=s.value))
        return bs

    bind_sets = [bindings_for(ci, co) for ci, co in zip(copies_in, copies_out)]
    kid = native.kernel_find(b.metal_function)
    launch = _async_launcher(name, b, copies_in, copies_out) if R > 1 else None
    torch.cuda.synchronize()
    if launch:
        def launch_n(count):
            for i in range(count):
                launch(i % R)
    else:
        def launch_n(count):
            native.run(kid, bind_sets[0], 0, count, native.RUN_WALL_ONLY)
    settled_ms = _settle(launch_n, settle_ms) if settle_ms > 0 else 0.0
    if warmup > 0:
        if launch:
            for i in range(warmup):
                launch(i % R)
        else:
            native.run(kid, bind_sets[0], 0, warmup, native.RUN_PIPELINED)
    # Timed region: exactly `steps` launches back to back, bracketed by
    # synchronize on both sides and by a hipEvent pair on the stream the
    # kernels run on (the library enqueues on torch's current stream here), so
    # the device time per launch is measured over the same region.
    stream = torch.cuda.Stream()   # default priority; a real (non-null) stream handle
    native.load().mb_set_stream(ctypes.c_void_p(stream.cuda_stream))
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    if launch:
        for i in range(steps):
            launch(i % R)
    else:
        native.run(kid, bind_sets[0], 0, steps, native.RUN_WALL_ONLY)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1000.0
    ms_per_step = wall_ms / steps
    device_ms = ev0.elapsed_time(ev1) / steps
    native.load().mb_set_stream(None)
    # Per-kernel durations (roofline): `steps` more steps with a hipEvent pair
    # per step and per-kernel events (the decode step's kernels carry their
    # own start and end events); rotating workloads run them one by one over
    # the copies, so each is timed cold as well.
    if R > 1:
        k_t = _mean_timing([native.run(kid, bind_sets[i % R], 0, 1,
                                       native.RUN_PIPELINED | native.RUN_PARTS)
                            for i in range(steps)])
    else:
        k_t = native.run(kid, bind_sets[0], 0, steps, native.RUN_PIPELINED | native.RUN_PARTS)
    torch.cuda.synchronize()

    k_t["device_ms_per_launch"] = device_ms
    w = _work(name, meta)
    value, unit, hib = _value_unit(name, meta, ms_per_step)
    rec = {"value": value, "unit": unit, "higher_is_better": hib, "ms_per_step": ms_per_step,
           "gpu_median_ms": k_t["median_ms"], "gpu_mean_ms": k_t["mean_ms"],
           "roofline": _roofline(name, w, k_t, b.compute_dtype), "dtype": b.compute_dtype,
           "cache": (f"cold: {R} rotating copies of the working set" if R > 1
                     else "warm: one set of buffers"),
           "clock_settle_ms": round(settled_ms, 1)}
    if k_t.get("parts"):
        rec["parts"] = [{"name": p["name"], "mean_us": p["mean_ms"] * 1e3,
                         **({"hbm_frac": w["parts"][p["name"]] / (p["mean_ms"] * 1e-3) / 1e9
                             / HBM_PEAK_GBPS} if "parts" in w and p["name"] in w["parts"] else {})}
                        for p in k_t["parts"]]
    del copies_in, copies_out
    torch.cuda.synchronize()
    if want_cpu:
        rec["cpu_baseline"] = _cpu_baseline(name, b, inputs, meta)
    return rec


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="llama_decoder_step")
    ap.add_argument("--only", action="store_true", help="skip the other configurations")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--settle-ms", type=float, default=100.0,
                    help="busy time with the workload's own launches before the W warmup "
                         "steps, so the timed steps run at the working clock (0: none)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run the 256 MiB copy kernel (counter calibration)")
    args = ap.parse_args(argv)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (every config fits one MI355X, and "
              "the multi-GPU sharding of the decode step is a design, not a run). Use --gpus 1.",
              file=sys.stderr)
        return 2

    import torch

    from metalbench_amd import native
    native.init(0)
    names = native.kernel_names()
    if args.copy_calibration:
        _copy_calibration()
    _measured_hbm_gbps()

    others = [n for n in ("transpose_2d", "sqr_mm", "conv2d", "large_mm") if n != args.workload]
    if args.only:
        others = []
    rank0 = True
    head = _run_workload(args.workload, args.steps, args.warmup, not args.no_cpu_baseline,
                         args.settle_ms)
    kernels = {}
    for n in others:
        from metalbench_amd import helpers as H
        fn = H.load_baseline(n).metal_function
        if fn not in names:
            kernels[n] = {"status": "not built"}
            continue
        print(f"[bench] {n} ...", file=sys.stderr, flush=True)
        kernels[n] = _run_workload(n, args.steps, args.warmup, not args.no_cpu_baseline,
                                   args.settle_ms)

    from metalbench_amd import helpers as H
    meta = H.load_baseline(args.workload).meta
    if args.workload in DECODE_STEPS:
        t = _step_shape(meta)
        config = {"workload": args.workload, "batch": t["B"], "kv_len": t["L"], "d_model": t["D"],
                  "n_heads": t["H"], "n_kv_heads": t["HKV"], "head_dim": t["DH"],
                  "d_ff": t["FF"], "rope_theta": 500000.0,
                  "parallelism": ("single-gpu" if args.workload == "llama_decoder_step" else
                                  "one GPU's share of 8-way tensor parallelism, all-reduces "
                                  "excluded")}
    else:
        config = {"workload": args.workload, "input_shapes": meta["input_shapes"],
                  "parallelism": "single-gpu"}
    line = {
        "metric": METRIC,
        "value": head["value"],
        "unit": head["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": head["higher_is_better"],
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head["dtype"],
        "data": "synthetic (seed 0; registry input_init distributions)",
        "config": config,
        "roofline": head["roofline"],
        "cache": head["cache"],
        "clock_settle_ms": head["clock_settle_ms"],
        "cpu_baseline": head.get("cpu_baseline"),
        "hbm_measured_gbps": _MEASURED_HBM.get("gbps"),
        "gpu_mean_ms": head["gpu_mean_ms"],
        "parts": head.get("parts"),
        "kernels": kernels,
        "device": torch.cuda.get_device_name(0),
    }
    if rank0:
        print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
