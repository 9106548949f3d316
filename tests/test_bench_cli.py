"""bench.py's command-line contract, checked without a GPU: more than one GPU is refused
with a message (this build measures one MI355X), and unknown workloads are rejected
before any device work."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120)


def test_more_than_one_gpu_is_refused():
    out = _bench("--gpus", "2")
    assert out.returncode == 2
    assert "--gpus 2 is not supported" in out.stderr
    assert out.stdout == ""  # no JSON line for a configuration that was not measured


def test_unknown_workload_is_rejected():
    out = _bench("--only", "c3,nope")
    assert out.returncode == 2
    assert "unknown workload nope" in out.stderr
