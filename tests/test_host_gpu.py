"""Device tests of the C++ host API (MatMul, Transpose, OptimizedGEMM, SparseMatMul,
SparseMatVec, FusedLinearActivation, ForwardFloat16, LinearLayer, GPUDense, GPUSparse)
through the C ABI, checked against the oracle. Runs the compiled test binary in --gpu
mode in one process."""
import importlib.util
import os

import pytest

from test_host_cpu import HERE, run_host_tests

pytestmark = pytest.mark.gpu


def _c1_fixture_writer():
    spec = importlib.util.spec_from_file_location("write_c1_fixture", os.path.join(HERE, "host", "write_c1_fixture.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.write


def test_host_api_gpu(tmp_path):
    # Config C1's committed fixture as raw arrays for TestGPUMatMulC1Golden.
    raw = tmp_path / "c1.bin"
    _c1_fixture_writer()(str(raw))
    os.environ["GONNGPU_C1_FIXTURE"] = str(raw)
    try:
        text = run_host_tests("--gpu")
    finally:
        del os.environ["GONNGPU_C1_FIXTURE"]
    for name in ("TestForwardFloat16", "TestGPUDenseTransposeViews", "TestGPUMatMulC1Golden"):
        assert f"--- PASS {name}" in text
    assert "--- FAIL" not in text
