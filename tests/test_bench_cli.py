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
    for w in ("cfg1", "cfg2", "cfg3", "cfg3layer", "cfg4", "cfg5", "decode_m1"):
        assert w in r.stdout


def test_no_device_is_a_clear_error():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a HIP device is present")
    r = run("--workload", "cfg1")
    assert r.returncode == 1
    assert "needs a HIP device" in r.stderr
