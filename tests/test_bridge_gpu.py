"""GPU checks of the reference-compatible buffer ABI and its error conventions
(internal/cgo/metal_bridge_buffer.m:24-86, metal_bridge_common.m:20-34)."""
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest

import gonngpu as G

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_buffer_roundtrip_and_partial_retrieve(dev):
    x = np.arange(1000, dtype=np.float32)
    b = G.Buffer.from_array(x)
    assert b.device is not None  # DevicePtr is a non-NULL context token
    np.testing.assert_array_equal(b.to_array((1000,)), x)
    np.testing.assert_array_equal(b.to_array((10,)), x[:10])  # shorter retrieve is allowed
    big = np.empty(1001, np.float32)
    rc, msg = G.call_rc("retrieve_gpu_buffer_data", b.handle, big.ctypes.data, big.nbytes)
    assert rc == -2 and "length mismatch" in msg
    b.release()
    rc, _ = G.call_rc("retrieve_gpu_buffer_data", b.handle, big.ctypes.data, 4)
    assert rc == -1  # released handle is no longer valid


def test_large_buffer_crosses_staging_chunks(dev):
    # 80 MB: three 32 MiB staging chunks, each host copy split over the copy threads, odd
    # size; then 3 MiB + 3 floats (one chunk, split copy with a ragged last slice)
    for n in (20_000_003, 786_435):
        x = np.random.default_rng(n).standard_normal(n).astype(np.float32)
        b = G.Buffer.from_array(x)
        np.testing.assert_array_equal(b.to_array(x.shape), x)
        b.release()


def test_zero_filled_buffer_and_stats(dev):
    cur0, peak0, n0 = G.memory_stats()
    b = G.Buffer(4096)
    assert np.all(b.to_array((1024,)) == 0)
    cur1, peak1, n1 = G.memory_stats()
    assert n1 == n0 + 1 and cur1 >= cur0 + 4096 and peak1 >= cur1
    b.release()
    assert G.memory_stats()[2] == n0


def test_matmul_dimension_errors(dev):
    a, b, c = G.Buffer(4 * 6), G.Buffer(4 * 6), G.Buffer(4 * 4)
    rc, _ = G.call_rc("perform_mps_matrix_multiplication", a.handle, 2, 3, b.handle, 2, 3, c.handle, 2, 3, None)
    assert rc == -3  # aCols != bRows
    rc, _ = G.call_rc("perform_mps_matrix_multiplication", None, 2, 3, b.handle, 3, 2, c.handle, 2, 2, None)
    assert rc == -2
    rc, _ = G.call_rc("perform_mps_matrix_multiplication", a.handle, 20, 30, b.handle, 30, 20, c.handle, 20, 20, None)
    assert rc == -3  # buffers too small for the claimed shapes
    # sizes whose byte counts wrap around 2^64 (2^40 * 2^40 * 4 = 2^82) are rejected before any launch
    big = 1 << 40
    rc, _ = G.call_rc("perform_mps_matrix_multiplication", a.handle, big, big, b.handle, big, 1 << 24, c.handle, big,
                      1 << 24, None)
    assert rc == -3
    rc, _ = G.call_rc("perform_batch_matmul_optimized", a.handle, b.handle, c.handle, 1 << 62, 4, 4, 4, None)
    assert rc == -3  # batch * M overflows
    rc, _ = G.call_rc("perform_mps_matrix_transpose", a.handle, big, big, b.handle, big, big, None)
    assert rc == -3


def test_optimized_gemm_alpha_beta(dev):
    rng = np.random.default_rng(2)
    A = rng.standard_normal((31, 45)).astype(np.float32)
    B = rng.standard_normal((45, 27)).astype(np.float32)
    C0 = rng.standard_normal((31, 27)).astype(np.float32)
    ba, bb, bc = G.Buffer.from_array(A), G.Buffer.from_array(B), G.Buffer.from_array(C0)
    G.call("perform_optimized_gemm", ba.handle, bb.handle, bc.handle, 31, 27, 45, 2.0, 0.5, None)
    ref = 2.0 * (A.astype(np.float64) @ B) + 0.5 * C0
    got = bc.to_array((31, 27))
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-5


def test_injected_allocation_failure_is_clean(dev):
    """GONNGPU_FAIL_ALLOC_AFTER makes the Nth device allocation fail; the call must
    return -3 with a message, and the process must keep working."""
    code = textwrap.dedent(f"""
        import sys
        sys.path.insert(0, {os.path.join(ROOT, 'go-nngpu_amd')!r})
        import numpy as np, gonngpu as G
        G.init()
        ok = G.Buffer.from_array(np.ones(16, np.float32))
        import ctypes
        h, d = ctypes.c_void_p(), ctypes.c_void_p()
        rc, msg = G.call_rc("create_gpu_buffer", None, 64, ctypes.byref(h), ctypes.byref(d))
        assert rc == -3 and "injected" in msg, (rc, msg)
        assert np.all(ok.to_array((16,)) == 1)
        print("OK")
    """)
    env = dict(os.environ, GONNGPU_FAIL_ALLOC_AFTER="1")
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and "OK" in out.stdout, out.stderr[-2000:]


def test_scratch_allocation_failure_is_clean(dev):
    """The GEMM's split-K partials and the SpMM's split positions live in a per-stream scratch
    block; when that allocation fails (injected) the call returns -3 with a message before
    anything is launched, and calls that need no scratch keep working."""
    code = textwrap.dedent(f"""
        import sys
        sys.path.insert(0, {os.path.join(ROOT, 'go-nngpu_amd')!r})
        import numpy as np, torch, gonngpu as G
        G.init()
        a = torch.randn(300, 8192, device="cuda").half()
        b = torch.randn(8192, 1000, device="cuda").half()
        c = torch.zeros(300, 1000, device="cuda")
        try:
            G.gemm(a, b, c)  # few tiles, long K: split-K, partials in the scratch
            raise SystemExit("split-K GEMM did not fail")
        except G.GonngpuError as e:
            assert e.code == -3 and "injected" in e.message, e
        M, K, N = 2000, 3000, 64
        rp = np.arange(0, 40 * (M + 1), 40, dtype=np.int32)
        col = np.tile(np.arange(0, 3000, 75, dtype=np.int32), M)
        val = np.ones(col.size, np.float32)
        d = [torch.from_numpy(x).cuda() for x in (rp, col, val)]
        D = torch.ones(K, N, device="cuda")
        C = torch.zeros(M, N, device="cuda")
        try:
            G.spmm_csr(M, N, K, val.size, d[0], d[1], d[2], D, C)  # 80000 entries: split positions in the scratch
            raise SystemExit("two-launch SpMM did not fail")
        except G.GonngpuError as e:
            assert e.code == -3 and "injected" in e.message, e
        x = torch.randn(64, 64, device="cuda")
        y = torch.empty(64, 64, device="cuda")
        G.gemm(x, x, y)  # no scratch needed
        torch.cuda.synchronize()
        assert torch.allclose(y, x @ x, rtol=1e-4, atol=1e-4)
        assert torch.count_nonzero(c).item() == 0 and torch.count_nonzero(C).item() == 0
        print("OK")
    """)
    env = dict(os.environ, GONNGPU_FAIL_ALLOC_AFTER="0")
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=180)
    assert out.returncode == 0 and "OK" in out.stdout, (out.stdout[-1000:], out.stderr[-2000:])


def test_release_is_stream_ordered(dev):
    """gn_free_async (and release_gpu_buffer, on the library stream) does not wait: a block
    freed while kernels on the library stream still read it goes to a new owner only after
    they have finished. Here A is freed right behind eight queued 4096^3 GEMMs that read it, a
    block of the same size is taken at once and overwritten from another stream; the GEMMs'
    output must still equal the product computed before. gn_free waits for the whole device
    instead: after it returns the block may be reused at once, and the GEMMs queued before it
    have finished."""
    import ctypes

    import torch

    n = 4096
    nbytes = n * n * 4

    def malloc():
        p = ctypes.c_void_p()
        G.call("gn_malloc", ctypes.byref(p), nbytes)
        return p.value

    pa = malloc()
    G.call("gn_fill_normal_f32", pa, n * n, 42, 901, 0.0, 1.0, None)
    B = torch.empty((n, n), dtype=torch.float32, device=dev)
    G.fill_normal(B, 42, 902)
    torch.cuda.synchronize()
    ref = torch.empty((n, n), dtype=torch.float32, device=dev)
    out = torch.empty((n, n), dtype=torch.float32, device=dev)

    def gemm(src, dst):  # on the library stream (NULL)
        G.call("gn_gemm", G.GN_F32, 0, 0, n, n, n, 1.0, src, n, 0, B.data_ptr(), n, 0, 0.0, dst.data_ptr(), n, 0, 1,
               None, G.ACT_NONE, 0.0, None)

    gemm(pa, ref)
    G.call("gn_synchronize", None)
    for _ in range(8):
        gemm(pa, out)
    G.call("gn_free_async", pa, None)  # A is still being read by the queued GEMMs
    pz = malloc()
    G.call("gn_fill_uniform_f32", pz, n * n, 7, 7, 100.0, 200.0, torch.cuda.current_stream().cuda_stream)
    G.call("gn_synchronize", None)
    torch.cuda.synchronize()
    assert pz != pa, "a block still read by queued kernels was handed out again"
    assert torch.equal(out, ref)
    # gn_free: device-wide wait, then the block is free at once
    G.call("gn_fill_normal_f32", pz, n * n, 42, 901, 0.0, 1.0, None)
    out.zero_()
    torch.cuda.synchronize()
    for _ in range(8):
        gemm(pz, out)
    G.call("gn_free", pz)
    p3 = malloc()
    G.call("gn_fill_uniform_f32", p3, n * n, 7, 7, 100.0, 200.0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(out, ref), "gn_free returned before the GEMMs reading the block had finished"
    # once the work is done, the freed blocks are reused (no growth of the pool)
    G.call("gn_free", p3)
    p2 = malloc()
    assert p2 in (pa, pz, p3)
    G.call("gn_free_async", p2, torch.cuda.current_stream().cuda_stream)
