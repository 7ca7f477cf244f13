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


def _bench_module():
    import importlib.util

    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_every_sample_times_exactly_steps_calls():
    """W untimed calls, then S samples of exactly K calls, each between two
    events and synchronisations; S >= 10 and S * K >= 1300."""
    from types import SimpleNamespace

    bench = _bench_module()
    log = []

    class Event:
        def __init__(self, enable_timing=False):
            self.t = None

        def record(self, stream=None):
            log.append("record")

        def elapsed_time(self, other):
            return 1.0

    fake = SimpleNamespace(cuda=SimpleNamespace(Event=Event, synchronize=lambda: log.append("sync")))
    calls = []
    for steps, warmup in ((20, 5), (240, 24), (1, 0)):
        calls.clear()
        log.clear()
        samples = bench.sample_plan(steps)
        assert samples >= 10 and samples * steps >= 1300
        ms = bench.timed_samples(fake, calls.append, steps, warmup, samples)
        assert calls == [warmup] + [steps] * samples and len(ms) == samples
        # each timed region: sync, record, calls, record, sync
        assert log.count("record") == 2 * samples and log.count("sync") >= 2 * samples
    assert bench.sample_plan(20) == 65 and bench.sample_plan(240) == 10


def test_sample_statistics():
    bench = _bench_module()
    st = bench.sample_stats([10.0] * 9 + [20.0])
    assert st["p50_us"] == 10.0 and st["p99_us"] == 20.0 and st["samples"] == 10
    assert not st["cv_ok"] and bench.sample_stats([10.0, 10.1, 9.9])["cv_ok"]


def test_cpu_baseline_rows_on_a_tiny_layer():
    """Both CPU rows (dequantize per call / pre-dequantized) on a small shape."""
    bench = _bench_module()
    from uma_qmoe_amd import synthetic as syn

    shape = syn.MoEShape("bench_tiny", 256, 8, 2, 128, 256)
    row, agreement = bench.cpu_baseline(shape, 0.2)
    assert agreement is None
    assert row["kind"] == "port" and row["cores"] >= 1 and row["value"] > 0
    assert row["predequantized"]["value"] > 0 and row["cpu_model"]


def test_counter_collection_is_refused():
    """Under rocprofv3 counter collection bench.py exits before touching a
    device (counters are taken with the standalone programs), except for the
    copy probe that calibrates them."""
    import os

    bench = _bench_module()
    assert bench.counter_collection_active({"ROCPROF_COUNTER_COLLECTION": "1"})
    assert bench.counter_collection_active({"ROCPROF_COUNTER_COLLECTION": "True"})
    assert bench.counter_collection_active({"ROCPROF_COUNTERS": "pmc: FETCH_SIZE"})
    assert not bench.counter_collection_active({"ROCPROF_COUNTER_COLLECTION": "0"})
    assert not bench.counter_collection_active({"ROCPROF_KERNEL_TRACE": "1"})
    env = dict(os.environ, ROCPROF_COUNTER_COLLECTION="True", ROCPROF_COUNTERS="pmc: FETCH_SIZE")
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--steps", "5"], cwd=ROOT, capture_output=True,
                       text=True, timeout=120, env=env)
    assert r.returncode == 3 and "counter collection" in r.stderr and r.stdout == ""
