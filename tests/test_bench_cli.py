"""bench.py's command line on the CPU: the one-GPU rule and the modes it offers."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _run(*args: str) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_more_than_one_gpu_exits_with_a_message():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""  # no JSON line for a run that did not happen


def test_modes_are_listed():
    r = _run("--help")
    assert r.returncode == 0
    for mode in ("bench", "pmc", "prefill", "decode", "ragged", "chunked"):
        assert mode in r.stdout


def test_cpu_baseline_helpers():
    sys.path.insert(0, str(ROOT))
    import bench

    assert bench.cpu_model()
    calls = []
    med, n = bench.time_cpu(lambda: calls.append(1), seconds=0.0, min_calls=5)
    assert n == 5 and len(calls) == 8 and med >= 0.0  # 3 warm-ups + 5 timed
