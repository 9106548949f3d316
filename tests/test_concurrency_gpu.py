"""Part-1 calls from several host threads at once (the Go side may call the bridge from
any goroutine; the reference's bridge initialises its globals lazily without
synchronisation, internal/cgo/metal_bridge_buffer.m:26-42). Eight threads create,
multiply, retrieve and release their own buffers concurrently through the C ABI (ctypes
releases the GIL during each call); every result is checked against the oracle."""
import threading

import numpy as np
import pytest

import gonngpu as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def test_part1_calls_from_eight_threads(dev):
    O.lib()  # load the checker once, before the threads share it
    G.init()
    errors = []
    barrier = threading.Barrier(8)

    def worker(t):
        try:
            rng = np.random.default_rng(100 + t)
            barrier.wait()
            for it in range(4):
                M, K, N = 64 + 32 * t, 96 + 16 * it, 80 + 8 * t
                A = rng.standard_normal((M, K)).astype(np.float32)
                B = rng.standard_normal((K, N)).astype(np.float32)
                ba, bb, bc = G.Buffer.from_array(A), G.Buffer.from_array(B), G.Buffer(M * N * 4)
                G.call("perform_mps_matrix_multiplication", ba.handle, M, K, bb.handle, K, N, bc.handle, M, N, None)
                C = bc.to_array((M, N))
                assert O.rel_frob(C, A.astype(np.float64) @ B.astype(np.float64)) <= 1e-5, ("gemm", t, it)
                rows, cols, W = 200 + t, 300, 32
                rp, col, val = O.random_csr(rows, cols, 6.0, seed=10 * t + it)
                D = O.normal((cols, W), t, it)
                bv, bd, bo = G.Buffer.from_array(val), G.Buffer.from_array(D), G.Buffer(rows * W * 4)
                for _ in range(2):  # the second call takes the cached index arrays
                    G.call("perform_sparse_dense_matmul", bv.handle, rp.ctypes.data, rp.size, col.ctypes.data,
                           col.size, rows, cols, val.size, bd.handle, cols, W, bo.handle, rows, W, None)
                    S = bo.to_array((rows, W))
                    assert np.array_equal(S, O.spmm_f32(rp, col, val, D, use_fma=True)), ("spmm", t, it)
                x = D[:, 0].copy()
                bx, by = G.Buffer.from_array(x), G.Buffer(rows * 4)
                G.call("perform_sparse_matvec", bv.handle, rp.ctypes.data, rp.size, col.ctypes.data, col.size, rows,
                       cols, val.size, bx.handle, cols, by.handle, rows, None)
                assert O.rel_frob(by.to_array((rows,)), O.spmv_f64(rp, col, val, x)) <= 1e-5, ("spmv", t, it)
                for b in (ba, bb, bc, bv, bd, bo, bx, by):
                    b.release()
        except Exception as e:  # reported by the main thread
            errors.append((t, repr(e)))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(8)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=240)
    assert not any(th.is_alive() for th in threads), "a worker thread did not finish"
    assert not errors, errors
