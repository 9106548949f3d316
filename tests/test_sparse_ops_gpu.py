"""GPU parity of the remaining sparse entry points through the C ABI (metal_bridge.h:
168-246) against the oracle's restatements of the reference loops
(internal/cgo/metal_bridge_sparse.m): sparse x sparse, dense x CSC, sparse add,
scalar multiply, CSR -> dense and dense -> COO. Every one follows the reference's order
per output, so results are compared bit for bit (fma variants of the restatements);
the products are also held to relFrob <= 1e-5 against float64."""
import ctypes
import sys

import numpy as np
import pytest

import gonngpu as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _p(a):
    return a.ctypes.data if a.size else None


def _rand_csr(rng, M, K, density, scale=1.0):
    D = np.where(rng.random((M, K)) < density, scale * rng.standard_normal((M, K)), 0.0).astype(np.float32)
    rows, cols = np.nonzero(D)
    rp = np.zeros(M + 1, np.int32)
    np.cumsum(np.bincount(rows, minlength=M), out=rp[1:])
    return D, rp, cols.astype(np.int32), np.ascontiguousarray(D[rows, cols])


def _spgemm(arp, acol, aval, bcp, brow, bval, M, K, N):
    ba = G.Buffer.from_array(aval) if aval.size else None
    bb = G.Buffer.from_array(bval) if bval.size else None
    bc = G.Buffer(max(M * N, 1) * 4)
    rc, msg = G.call_rc("perform_sparse_sparse_matmul", ba.handle if ba else None, _p(arp), arp.size, _p(acol),
                        acol.size, M, K, aval.size, bb.handle if bb else None, _p(bcp), bcp.size, _p(brow), brow.size,
                        K, N, bval.size, bc.handle, M, N, None)
    return rc, msg, (bc.to_array((M, N)) if rc == 0 else None)


@pytest.mark.parametrize("M,K,N,da,db", [(64, 96, 80, 0.1, 0.1), (300, 500, 257, 0.02, 0.05), (1, 7, 1, 0.9, 0.9)])
def test_sparse_sparse_matmul(dev, M, K, N, da, db):
    rng = np.random.default_rng(301 + M)
    A, arp, acol, aval = _rand_csr(rng, M, K, da)
    Bd, brp, bcol, bval = _rand_csr(rng, K, N, db)
    bcp, brow, bv = O.csr_to_csc(K, N, brp, bcol, bval)
    rc, msg, C = _spgemm(arp, acol, aval, bcp, brow, bv, M, K, N)
    assert rc == 0, msg
    np.testing.assert_array_equal(C, O.spgemm_csr_csc_f32(arp, acol, aval, bcp, brow, bv))
    assert O.rel_frob(C, A.astype(np.float64) @ Bd.astype(np.float64)) <= 1e-5


def test_sparse_sparse_matmul_edges(dev):
    one = lambda *v: np.array(v, np.int32)
    f32 = lambda *v: np.array(v, np.float32)
    # duplicates pair in merge order (2*5 + 3*7), a cancelling pair stores +0
    rc, _, C = _spgemm(one(0, 2, 4), one(1, 1, 0, 1), f32(2, 3, 1, -1), one(0, 2, 4), one(1, 1, 0, 1),
                       f32(5, 7, 1, 1), 2, 2, 2)
    assert rc == 0 and C[0, 0] == 31.0 and C[1, 1] == 0.0 and not np.signbit(C[1, 1])
    # nnz = 0 on both sides: zeros (NULL value buffers allowed)
    rc, _, C = _spgemm(np.zeros(4, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32), np.zeros(6, np.int32),
                       np.zeros(0, np.int32), np.zeros(0, np.float32), 3, 4, 5)
    assert rc == 0 and not C.any()
    # malformed row pointers -> -3; inner dimension mismatch -> -2
    rc, msg, _ = _spgemm(one(0, 3, 1), one(0, 1, 2), f32(1, 1, 1), one(0, 1), one(0), f32(1), 2, 3, 1)
    assert rc == -3, msg
    ba, bc = G.Buffer.from_array(f32(1)), G.Buffer(16)
    rc, _ = G.call_rc("perform_sparse_sparse_matmul", ba.handle, one(0, 1).ctypes.data, 2, one(0).ctypes.data, 1, 1,
                      3, 1, ba.handle, one(0, 1).ctypes.data, 2, one(0).ctypes.data, 1, 4, 1, 1, bc.handle, 1, 1, None)
    assert rc == -2


def _dense_sparse(A, bcp, brow, bval, K, N):
    M = A.shape[0]
    ba = G.Buffer.from_array(A)
    bb = G.Buffer.from_array(bval) if bval.size else None
    bc = G.Buffer(max(M * N, 1) * 4)
    rc, msg = G.call_rc("perform_dense_sparse_matmul", ba.handle, M, A.shape[1], bb.handle if bb else None, _p(bcp),
                        bcp.size, _p(brow), brow.size, K, N, bval.size, bc.handle, M, N, None)
    return rc, msg, (bc.to_array((M, N)) if rc == 0 else None)


@pytest.mark.parametrize("M,K,N,d", [(512, 1024, 768, 0.02), (7, 33, 129, 0.2), (64, 64, 64, 0.0)])
def test_dense_sparse_matmul(dev, M, K, N, d):
    rng = np.random.default_rng(311 + M)
    A = rng.standard_normal((M, K)).astype(np.float32)
    Bd, brp, bcol, bval = _rand_csr(rng, K, N, d)
    bcp, brow, bv = O.csr_to_csc(K, N, brp, bcol, bval)
    rc, msg, C = _dense_sparse(A, bcp, brow, bv, K, N)
    assert rc == 0, msg
    np.testing.assert_array_equal(C, O.dense_csc_f32(A, bcp, brow, bv))
    if d > 0:
        assert O.rel_frob(C, A.astype(np.float64) @ Bd.astype(np.float64)) <= 1e-5
    else:
        assert not C.any()


def test_dense_sparse_matmul_bad_row_index(dev):
    A = np.ones((4, 5), np.float32)
    bcp, brow, bval = np.array([0, 1, 2], np.int32), np.array([1, 9], np.int32), np.ones(2, np.float32)
    rc, msg, _ = _dense_sparse(A, bcp, brow, bval, 5, 2)
    assert rc == -3, msg


def _sparse_add(arp, acol, aval, brp, bcol, bval, M, N, cap=None):
    cap = aval.size + bval.size if cap is None else cap
    ri, ci, vv = np.zeros(max(cap, 1), np.int32), np.zeros(max(cap, 1), np.int32), np.zeros(max(cap, 1), np.float32)
    n = ctypes.c_long(-1)
    ba = G.Buffer.from_array(aval) if aval.size else None
    bb = G.Buffer.from_array(bval) if bval.size else None
    rc, msg = G.call_rc("perform_sparse_add", ba.handle if ba else None, _p(arp), arp.size, _p(acol), acol.size, M, N,
                        aval.size, bb.handle if bb else None, _p(brp), brp.size, _p(bcol), bcol.size, M, N, bval.size,
                        ri.ctypes.data, ci.ctypes.data, vv.ctypes.data, ctypes.byref(n), cap, None)
    return rc, msg, ri[:max(n.value, 0)], ci[:max(n.value, 0)], vv[:max(n.value, 0)]


@pytest.mark.parametrize("M,N,d", [(25, 33, 0.3), (2000, 3000, 0.01), (5, 4, 0.0)])
def test_sparse_add(dev, M, N, d):
    rng = np.random.default_rng(321 + M)
    A, arp, acol, aval = _rand_csr(rng, M, N, d)
    B, brp, bcol, bval = _rand_csr(rng, M, N, d)
    # exact cancellations where both have an entry
    for i, j in np.argwhere((A != 0) & (B != 0))[:7]:
        bval[np.searchsorted(bcol[brp[i]:brp[i + 1]], j) + brp[i]] = -A[i, j]
    rc, msg, ri, ci, vv = _sparse_add(arp, acol, aval, brp, bcol, bval, M, N)
    assert rc == 0, msg
    orc = O.sparse_add(arp, acol, aval, brp, bcol, bval)
    assert orc[0] == 0
    np.testing.assert_array_equal(ri, orc[1])
    np.testing.assert_array_equal(ci, orc[2])
    np.testing.assert_array_equal(vv, orc[3])
    if ri.size:
        rc2, msg2, *_ = _sparse_add(arp, acol, aval, brp, bcol, bval, M, N, cap=ri.size - 1)
        assert rc2 == -2, msg2


def test_sparse_add_errors(dev):
    one = lambda *v: np.array(v, np.int32)
    v1 = np.ones(1, np.float32)
    rc, _, *_ = _sparse_add(one(0, 1), one(7), v1, one(0, 1), one(0), v1, 1, 3)
    assert rc == -3  # column outside [0, cols)
    ba = G.Buffer.from_array(v1)
    n = ctypes.c_long(0)
    out = np.zeros(4, np.int32)
    rc, _ = G.call_rc("perform_sparse_add", ba.handle, one(0, 1).ctypes.data, 2, one(0).ctypes.data, 1, 1, 3, 1,
                      ba.handle, one(0, 1, 1).ctypes.data, 3, one(0).ctypes.data, 1, 2, 3, 1, out.ctypes.data,
                      out.ctypes.data, out.ctypes.data, ctypes.byref(n), 4, None)
    assert rc == -1  # dimensions differ


def test_sparse_scalar_multiply(dev):
    rng = np.random.default_rng(331)
    v = rng.standard_normal(100003).astype(np.float32)
    b = G.Buffer.from_array(v)
    rp = np.array([0, v.size], np.int32)
    ci = np.zeros(v.size, np.int32)
    G.call("perform_sparse_scalar_multiply", b.handle, rp.ctypes.data, 2, ci.ctypes.data, v.size, 1, 1, v.size,
           np.float32(-2.5), None)
    np.testing.assert_array_equal(b.to_array(v.shape), v * np.float32(-2.5))


def test_sparse_to_dense(dev):
    rng = np.random.default_rng(341)
    M, N = 300, 200
    _, rp, ci, vv = _rand_csr(rng, M, N, 0.05)
    # duplicates (unsorted) in row 3: the later one wins
    rp2 = rp.copy()
    ci2 = np.insert(ci, rp[4], [5, 5])
    vv2 = np.insert(vv, rp[4], np.array([1.5, -2.5], np.float32))
    rp2[4:] += 2
    bv, bd = G.Buffer.from_array(vv2), G.Buffer(M * N * 4)
    G.call("perform_sparse_to_dense", bv.handle, rp2.ctypes.data, rp2.size, ci2.ctypes.data, ci2.size, M, N, vv2.size,
           bd.handle, M, N, None)
    D = bd.to_array((M, N))
    np.testing.assert_array_equal(D, O.csr_to_dense(M, N, rp2, ci2, vv2))
    assert D[3, 5] == -2.5
    rc, _ = G.call_rc("perform_sparse_to_dense", bv.handle, rp2.ctypes.data, rp2.size, ci2.ctypes.data, ci2.size, M,
                      N, vv2.size, bd.handle, M, N + 1, None)
    assert rc == -1  # dimension mismatch
    bad = ci2.copy()
    bad[0] = N
    rc, msg = G.call_rc("perform_sparse_to_dense", bv.handle, rp2.ctypes.data, rp2.size, bad.ctypes.data, bad.size, M,
                        N, vv2.size, bd.handle, M, N, None)
    assert rc == -3 and "column" in msg


@pytest.mark.parametrize("M,N,thr", [(17, 29, 0.5), (2000, 3000, 2.0), (3, 130, 0.0)])
def test_dense_to_sparse(dev, M, N, thr):
    rng = np.random.default_rng(351 + M)
    D = rng.standard_normal((M, N)).astype(np.float32)
    D[0, 1] = np.nan
    D[M - 1, N - 1] = -np.inf
    bd = G.Buffer.from_array(D)
    cap = M * N
    ri, ci, vv = np.zeros(cap, np.int32), np.zeros(cap, np.int32), np.zeros(cap, np.float32)
    n = ctypes.c_long(-1)
    G.call("perform_dense_to_sparse", bd.handle, M, N, np.float32(thr), ri.ctypes.data, ci.ctypes.data,
           vv.ctypes.data, ctypes.byref(n), cap, None)
    rc, r2, c2, v2 = O.dense_to_coo(D, thr)
    assert rc == 0 and n.value == r2.size
    np.testing.assert_array_equal(ri[:n.value], r2)
    np.testing.assert_array_equal(ci[:n.value], c2)
    np.testing.assert_array_equal(vv[:n.value], v2)
    rc, msg = G.call_rc("perform_dense_to_sparse", bd.handle, M, N, np.float32(thr), ri.ctypes.data, ci.ctypes.data,
                        vv.ctypes.data, ctypes.byref(n), max(r2.size - 1, 0), None)
    assert rc == -2, msg
