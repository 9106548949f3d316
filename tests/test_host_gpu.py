"""Device tests of the C++ host API (MatMul, Transpose, OptimizedGEMM, SparseMatMul,
SparseMatVec, FusedLinearActivation, ForwardFloat16, LinearLayer, GPUDense, GPUSparse)
through the C ABI, checked against the oracle. Runs the compiled test binary in --gpu
mode in one process."""
import pytest

from test_host_cpu import run_host_tests

pytestmark = pytest.mark.gpu


def test_host_api_gpu():
    text = run_host_tests("--gpu")
    assert "--- PASS TestForwardFloat16" in text
    assert "--- FAIL" not in text
