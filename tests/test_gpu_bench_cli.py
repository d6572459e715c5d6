"""Every registry entry through the user-facing CLI on the GPU: `./bench <name>`
runs the harness in a fresh process, which must print `correctness : ✓` with
max_err <= 0.05 and exit 0 -- the reference's accuracy sweep
(reference tests/metalbench/test_bench_accuracy_all.py:16-54, regex :32,
5 % bar :17), here against the registry's torch-CPU Model spec.  Unlike the
parity tests (which compare with the float64 oracle), this exercises
harness.evaluate(), the spec, the tolerance gate and the exit code."""
from __future__ import annotations

import os
import re
import subprocess

import pytest

from metalbench_amd import helpers as H

pytestmark = pytest.mark.gpu

REPO = H.REPO_ROOT
RTOL = 0.05
_RX_CORRECT = re.compile(r"correctness\s+:\s*(✓|✗).*?max_err=([\d.eE+-]+)")


def _discover_kernels() -> list[tuple[str, str]]:
    out = []
    for s in ("common", "standard", "full"):
        reg = REPO / "mlx" / "kernels" / s / "registry.py"
        if not reg.is_file():
            continue
        ns: dict = {}
        exec(reg.read_text(), ns)
        out += [(s, k) for k in sorted(ns.get("REGISTRY", {}))]
    return out


@pytest.mark.parametrize("set_name,kernel", _discover_kernels())
def test_kernel_accuracy_within_5pct(set_name, kernel):
    print(f"[cli] ./bench {kernel}", flush=True)
    env = dict(os.environ, SKIP_BUILD="1")   # test the library as built, never rebuild here
    r = subprocess.run(["./bench", kernel, "--no-save", "--", "--no-session", "--iters", "5",
                        "--warmup", "2", "--cpu-iters", "1"],
                       cwd=REPO, capture_output=True, text=True, timeout=300, env=env)
    out = r.stdout + r.stderr
    m = _RX_CORRECT.search(out)
    assert m, f"{set_name}/{kernel}: no correctness line (exit {r.returncode}):\n{out[-2000:]}"
    ok, err = m.group(1) == "✓", float(m.group(2))
    assert ok, f"{set_name}/{kernel}: correctness failed (max_err={err})\n{out[-2000:]}"
    assert err <= RTOL, f"{set_name}/{kernel}: max_err={err:.4e} > {RTOL}"
    assert r.returncode == 0, f"{set_name}/{kernel}: exit {r.returncode}\n{out[-2000:]}"
