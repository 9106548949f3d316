"""bench.py's command-line contract, checked without a GPU: more than one GPU is refused
with a message (this build measures one MI355X), and unknown workloads are rejected
before any device work."""
import json
import os
import subprocess
import sys

import pytest

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


@pytest.mark.gpu
def test_mfma_ceiling_probe(dev):
    """The bench's ceiling leg: the probe executable (run as a child process, as bench.py runs
    it) prints one JSON object whose two rates are plausible for one MI355X: within the
    2516.6 TFLOP/s spec peak, and the all-zero operands no slower than the benchmark's."""
    exe = os.path.join(ROOT, "go-nngpu_amd", "lib", "mfma_ceiling")
    out = subprocess.run([exe, "0.3"], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    res = json.loads(out.stdout.strip().splitlines()[-1])
    g, z = res["gemm_data"]["tflops"], res["zero_data"]["tflops"]
    assert 300.0 < g <= 2516.6 * 1.02 and 300.0 < z <= 2516.6 * 1.02, (g, z)
    assert z >= 0.9 * g, (g, z)
