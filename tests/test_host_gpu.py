"""Device tests of the C++ host API (MatMul, Transpose, OptimizedGEMM, SparseMatMul,
SparseMatVec, FusedLinearActivation, ForwardFloat16, LinearLayer, GPUDense, GPUSparse)
through the C ABI, checked against the oracle. Runs the compiled test binary in --gpu
mode in one process."""
import os

import numpy as np
import pytest

from test_host_cpu import HERE, run_host_tests

pytestmark = pytest.mark.gpu


def test_host_api_gpu(tmp_path):
    # Config C1's committed fixture as raw arrays for TestGPUMatMulC1Golden.
    z = np.load(os.path.join(HERE, "golden", "gemm_256.npz"))
    raw = tmp_path / "c1.bin"
    with open(raw, "wb") as f:
        f.write(np.ascontiguousarray(z["A"], dtype=np.float32).tobytes())
        f.write(np.ascontiguousarray(z["B"], dtype=np.float32).tobytes())
        f.write(np.ascontiguousarray(z["C64"], dtype=np.float64).tobytes())
    os.environ["GONNGPU_C1_FIXTURE"] = str(raw)
    try:
        text = run_host_tests("--gpu")
    finally:
        del os.environ["GONNGPU_C1_FIXTURE"]
    for name in ("TestForwardFloat16", "TestGPUDenseTransposeViews", "TestGPUMatMulC1Golden"):
        assert f"--- PASS {name}" in text
    assert "--- FAIL" not in text
