"""bench.py's command-line contract on a host without a GPU: one GPU only (--gpus N > 1 exits
with a message), the workload names, and a clear refusal without a HIP device."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run(*args, env=None):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=300, env=env)


def test_more_than_one_gpu_is_refused():
    r = run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU only" in r.stderr


def test_world_size_above_one_is_refused():
    env = dict(os.environ, WORLD_SIZE="2")
    r = run(env=env)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr


def test_unknown_workload_is_rejected():
    r = run("--workload", "cfg9")
    assert r.returncode == 2
    assert "invalid choice" in r.stderr


def test_workloads_listed_in_help():
    r = run("--help")
    assert r.returncode == 0
    for w in ("cfg1", "cfg2", "cfg3", "cfg3layer", "cfg4", "cfg5", "decode_m1", "prefill"):
        assert w in r.stdout


def test_no_device_is_a_clear_error():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a HIP device is present")
    r = run("--workload", "cfg1")
    assert r.returncode == 1
    assert "needs a HIP device" in r.stderr


def _bench_module():
    import importlib.util
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_step_stats_median_and_spread():
    """The per-step summary beside the mean: median of an even and an odd count, min, max."""
    b = _bench_module()
    b.STEP_TIMES[:] = [0.9, 0.7, 0.8, 1.3]
    s = b.step_stats()
    assert s == {"ms_per_step_median": 0.85, "ms_per_step_min": 0.7, "ms_per_step_max": 1.3,
                 "per_step_samples": 4}
    b.STEP_TIMES[:] = [2.0, 0.5, 1.0]
    assert b.step_stats()["ms_per_step_median"] == 1.0
    b.STEP_TIMES[:] = []
    assert b.step_stats() == {}
