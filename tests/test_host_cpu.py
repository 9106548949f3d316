"""Host-only tests of the C++ host API (go-nngpu_amd/host/gometal.hpp): tensor and
sparse-tensor construction, validation errors, COO->CSR/CSC, fp16 bit conversion,
gonum Dense and GPUSparse.At. Runs the compiled test binary in --cpu mode."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
BIN = os.path.join(HERE, "host", "_build", "test_host")


def build_host_tests():
    jobs = str(min(16, os.cpu_count() or 1))
    subprocess.run(["make", "-s", "-j", jobs, "-C", os.path.join(ROOT, "go-nngpu_amd")], check=True)
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "liboracle.so"], check=True)
    subprocess.run(["make", "-s", "-C", os.path.join(HERE, "host")], check=True)


def run_host_tests(mode):
    if not os.path.exists(BIN):
        build_host_tests()
    out = subprocess.run([BIN, mode], capture_output=True, text=True, timeout=600)
    print(out.stdout)
    assert out.returncode == 0, out.stdout[-4000:] + out.stderr[-2000:]
    return out.stdout


def test_host_api_cpu():
    text = run_host_tests("--cpu")
    assert "--- PASS TestConvertToCSRMatchesOracle" in text
    assert "--- FAIL" not in text
