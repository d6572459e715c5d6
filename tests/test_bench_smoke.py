"""Smoke asserts for ./bench and bench.py that need no GPU (reference
tests/metalbench/test_bench_smoke.py:12-34)."""
import json
import subprocess
import sys

from metalbench_amd import helpers as H

REPO = H.REPO_ROOT


def test_bench_script_is_executable():
    p = REPO / "bench"
    assert p.is_file() and (p.stat().st_mode & 0o111)


def test_bench_help_runs():
    r = subprocess.run(["./bench", "--help"], cwd=REPO, capture_output=True, text=True, timeout=10)
    assert "usage" in (r.stdout + r.stderr).lower()


def test_session_json_parses_if_present():
    p = REPO / "session.json"
    if p.exists():
        assert isinstance(json.loads(p.read_text()), dict)


def test_bench_py_refuses_multi_gpu():
    r = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], cwd=REPO,
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "one GPU" in r.stderr
