"""`--profile` and the kernel trace (`--xcode` / `--gputracer` /
`--capture-host`) through the user-facing CLI on the GPU.

The reference samples hardware counters around one extra dispatch and prints
them as the report's `profiling` block (reference mlx/scripts/harness.py:401-402,
322-326; metal/scripts/main.mm:53-71), and records a trace of one extra
dispatch (harness.py:395-400, 455-476; metal/scripts/timing.mm:199-229).  Here
both run that dispatch again in a child process under rocprofv3.  Each case
runs `./bench` in a fresh process with SKIP_BUILD=1, so the library is tested
as built."""
from __future__ import annotations

import os
import re
import subprocess
from pathlib import Path

import pytest

from metalbench_amd import helpers as H

pytestmark = pytest.mark.gpu

REPO = H.REPO_ROOT
_RX_SAMPLE = re.compile(r"^\s{4}([A-Z][A-Z0-9_]+)\s+(\d+)\s*$", re.M)


def _bench(*argv, timeout=300):
    print(f"[cli] ./bench {' '.join(argv)}", flush=True)
    env = dict(os.environ, SKIP_BUILD="1")
    r = subprocess.run(["./bench", *argv], cwd=REPO, capture_output=True, text=True,
                       timeout=timeout, env=env)
    return r, r.stdout + r.stderr


def _samples(out: str) -> dict:
    block = out.split("  profiling   : rocprofv3 --pmc (", 1)
    assert len(block) == 2, f"no profiling block:\n{out[-3000:]}"
    return {k: int(v) for k, v in _RX_SAMPLE.findall(block[1])}


def test_profile_sqr_mm_mfma_busy_cycles_closed_form():
    """Every fp32 MFMA retires 64 flop per SIMD-cycle (256 per CU-clock), so
    the 1024^3 GEMM's 2^31 flop keep the MFMA pipe busy for exactly
    2^31 / 64 = 2^25 cycles, whatever the tile shape (1024 is a multiple of
    every tile, so no MFMA works on padding)."""
    r, out = _bench("sqr_mm", "--no-save", "--", "--no-session", "--profile",
                    "--iters", "5", "--warmup", "2", "--cpu-iters", "1")
    assert r.returncode == 0, out[-3000:]
    assert "correctness : ✓" in out
    s = _samples(out)
    assert s["SQ_VALU_MFMA_BUSY_CYCLES"] == 2 ** 25, s
    assert s["SQ_INSTS_MFMA"] > 0 and s["GRBM_GUI_ACTIVE"] > 0
    # the counter-set line lists what the passes sample
    assert re.search(r"^  counters    : GRBM_GUI_ACTIVE, .*WRITE_SIZE$", out, re.M), out[-3000:]


def test_profile_decoder_step_hbm_traffic():
    """The decode step streams 570,753,024 algorithmic bytes (weights, KV cache,
    x, y and the new k, v); the one profiled dispatch is the first of its
    process, so L2 holds none of it and its L2-miss reads are at least nearly
    all of it.  On gfx950 FETCH_SIZE counts those reads at half their bytes:
    a plain copy of 256 MiB reads 131,088 KiB (READ_SCALE 2, the calibration
    bench.py --copy-calibration measures).  The step's workspace traffic (split-K
    partials) and the prefetched weight units that later kernels fetch again
    keep the total below 1.2x of the algorithmic bytes."""
    READ_SCALE = 2.0
    r, out = _bench("llama_decoder_step", "--no-save", "--", "--no-session", "--profile",
                    "--iters", "3", "--warmup", "1", "--cpu-iters", "1")
    assert r.returncode == 0, out[-3000:]
    s = _samples(out)
    fetch_bytes = s["FETCH_SIZE"] * 1024 * READ_SCALE
    assert 0.95 * 570_753_024 <= fetch_bytes <= 1.3 * 570_753_024, s
    # y, k_new and v_new at least (WRITE_SIZE counts whole bytes)
    assert s["WRITE_SIZE"] * 1024 >= 2 * (16 * 4096 + 2 * 16 * 8 * 128), s


def test_xcode_trace_of_decoder_step_names_its_five_kernels():
    r, out = _bench("llama_decoder_step", "--xcode", "--", "--no-session",
                    "--iters", "3", "--warmup", "1", "--cpu-iters", "1")
    assert r.returncode == 0, out[-3000:]
    m = re.search(r"\[host\] trace written: (\S+)", out)
    assert m, out[-3000:]
    trace_dir = m.group(1)
    assert trace_dir.endswith("llama_decoder_step.trace")
    assert list(Path(trace_dir).rglob("*_kernel_trace.csv"))
    body = out.split("  trace       : ", 1)[1]
    rows = re.findall(r"^    (\S.*?)\s+([\d.]+) µs$", body, re.M)
    assert len(rows) == 5, body[:2000]
    assert all(float(us) > 0 for _, us in rows)


def test_gputracer_one_entry_into_capture_dir(tmp_path):
    cap = tmp_path / "tr"
    r, out = _bench("--gputracer", "transpose_2d", "--capture-host", str(cap),
                    "--no-session", "--iters", "3", "--warmup", "1", "--cpu-iters", "1")
    assert r.returncode == 0, out[-3000:]
    assert f"[host] trace written: {cap}" in out
    assert list(cap.rglob("transpose_2d_kernel_trace.csv"))
    assert re.search(r"^    \S*transpose\S*\s+[\d.]+ µs$", out, re.M), out[-3000:]
