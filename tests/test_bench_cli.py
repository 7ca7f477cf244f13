"""bench.py's command-line contract, checked without a GPU: more than one GPU
is refused before anything touches a device, and the flags the profiles'
commands use exist."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def run_bench(*args: str) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT, capture_output=True, text=True,
                          timeout=120)


def test_more_than_one_gpu_is_refused():
    r = run_bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in (r.stdout + r.stderr)


def test_profile_command_flags_exist():
    r = run_bench("--help")
    assert r.returncode == 0
    for flag in ("--tokens", "--config", "--no-cpu-baseline", "--no-batch32", "--multi-kernel", "--copy-probe",
                 "--steps", "--warmup"):
        assert flag in r.stdout, flag
