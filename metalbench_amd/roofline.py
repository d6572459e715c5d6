"""Roofline classification against the MI355X (gfx950) datasheet peaks.

Same interface and classification rule as reference mlx/scripts/roofline.py:28-82
(compute-bound above the ridge, balanced within half of it, memory-bound below;
latency-dominated under 50 us).  The difference: MI355X has one HBM peak but a
different matrix-core peak per dtype, so `classify` takes the dtype the kernel
computes in.

Peaks (AMD public datasheet; dense, no sparsity): HBM3E 8.0 TB/s; matrix cores
fp32 157.3, bf16/fp16 2516.6, fp8 5033.2 TFLOP/s; fp64 78.6 TFLOP/s.
256 CUs at 2.4 GHz.
"""

CHIP_PEAKS = {
    "gfx950": dict(bw_GBps=8000.0, compute_TFLOPS=157.3,
                   compute_TFLOPS_by_dtype={"f32": 157.3, "bf16": 2516.6, "f16": 2516.6,
                                            "fp8": 5033.2, "f64": 78.6}),
}


def peak_for(chip_type: str, dtype: str = "f32") -> dict:
    peak = CHIP_PEAKS.get(chip_type.split(":")[0], CHIP_PEAKS["gfx950"])
    tf = peak["compute_TFLOPS_by_dtype"].get(dtype, peak["compute_TFLOPS"])
    return dict(bw_GBps=peak["bw_GBps"], compute_TFLOPS=tf, dtype=dtype)


def classify(chip_type: str, flops: float, bytes_: float, median_ms: float, dtype: str = "f32"):
    peak = peak_for(chip_type, dtype)
    intensity = (flops / bytes_) if bytes_ > 0 else 0.0
    ridge = peak["compute_TFLOPS"] * 1000.0 / peak["bw_GBps"]

    seconds = median_ms / 1000.0
    gflops = (flops / seconds / 1e9) if seconds > 0 else 0.0
    gbps = (bytes_ / seconds / 1e9) if seconds > 0 else 0.0

    sol_compute = gflops / (peak["compute_TFLOPS"] * 1000.0)
    sol_memory = gbps / peak["bw_GBps"]

    if flops == 0:
        cls, sol = "memory-bound", sol_memory
    elif intensity > ridge:
        cls, sol = "compute-bound", sol_compute
    elif intensity > ridge * 0.5:
        cls, sol = "balanced", max(sol_compute, sol_memory)
    else:
        cls, sol = "memory-bound", sol_memory

    if median_ms < 0.05:
        cls = cls + " (latency-dominated <50µs)"

    if cls.startswith("memory"):
        suggest = "16-byte coalesced loads, more bytes in flight per CU, fewer HBM passes"
    elif cls.startswith("compute"):
        suggest = "bigger MFMA tiles, LDS double-buffering, conflict-free ds_read, XCD-aware tile order"
    else:
        suggest = "overlap loads with MFMA, larger tile — already near both ceilings"
    if "latency" in cls:
        suggest = "launch/latency dominates — more work per launch, fewer kernels per step"

    return dict(intensity=intensity, ridge=ridge, gflops=gflops, gbps=gbps, sol=sol,
                sol_compute=sol_compute, sol_memory=sol_memory, classification=cls,
                suggest=suggest, peak=peak)


def format_line(metrics) -> str:
    return (
        f"  roofline    : {metrics['classification']}  "
        f"sol={metrics['sol']*100:.0f}%  "
        f"intensity={metrics['intensity']:.2f} vs ridge {metrics['ridge']:.1f}\n"
        f"              {metrics['suggest']}"
    )
