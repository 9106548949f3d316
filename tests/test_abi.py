"""CPU checks of the C ABI: the library builds/loads and exports every entry point
that include/gonngpu.h declares (no device work is done here)."""
import ctypes
import os
import re
import subprocess

import pytest

import gonngpu as G

# Declared in the reference bridge (internal/cgo/metal_bridge.h) and re-exported unchanged.
REFERENCE_NAMES = {
    "create_gpu_buffer", "retrieve_gpu_buffer_data", "release_gpu_buffer", "perform_mps_matrix_multiplication",
    "perform_mps_matrix_transpose", "perform_optimized_gemm", "perform_batch_matmul_optimized",
    "perform_fused_linear_activation", "perform_sparse_dense_matmul", "perform_sparse_matvec",
    "free_c_error_message",
}


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(G.LIB_PATH):
        subprocess.run(["make", "-s", "-j", str(min(16, os.cpu_count() or 1)), "-C", G.PKG_DIR], check=True)
    return G.load()


def test_header_declares_reference_subset_and_extensions():
    names = set(G.header_symbols())
    assert REFERENCE_NAMES <= names
    assert {n for n in names if n.startswith("gn_")} >= {"gn_gemm", "gn_spmm_csr", "gn_spmv_csr", "gn_cast_f32_f16"}


def test_library_exports_every_declared_symbol(lib):
    for name in G.header_symbols():
        assert hasattr(lib, name), f"{name} declared in include/gonngpu.h but not exported"
    assert set(G.SIGNATURES) <= set(G.header_symbols()), "ctypes table binds an undeclared name"


def test_library_targets_gfx950_only(lib):
    # The embedded offload bundle names its code-object targets; all must be gfx950.
    blob = open(G.LIB_PATH, "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa-[-\w:+]*gfx\d+", blob))
    assert targets == {b"amdgcn-amd-amdhsa--gfx950"}, targets


def test_version_string(lib):
    assert b"gfx950" in lib.gn_version()


def test_free_c_error_message_accepts_null(lib):
    lib.free_c_error_message(None)


def test_release_null_is_noop(lib):
    assert lib.release_gpu_buffer(None) == 0


def test_invalid_handle_rejected_without_device(lib):
    # An unknown handle is rejected before any device call.
    bogus = ctypes.c_void_p(0x1234)
    assert lib.gn_buffer_bytes(bogus) == -1
    assert lib.gn_buffer_device_ptr(bogus) is None


def test_spmv_dimension_check_precedes_device(lib):
    # metal_bridge_sparse.m:306-309: dimension mismatch is reported as -1 before buffers are touched.
    rc, msg = G.call_rc("perform_sparse_matvec", None, None, 1, None, 0, 0, 5, 0, None, 4, None, 0, None)
    assert rc == -1 and "Incompatible dimensions" in msg
