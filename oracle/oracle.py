"""ctypes front-end for the CPU checker in oracle.c.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker, never as the thing measured
or shipped. The product path (go-nngpu_amd/) never imports this module.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_L = ctypes.c_long
_U64 = ctypes.c_uint64


def build():
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    L = ctypes.CDLL(_LIB_PATH)
    sig = {
        "orc_splitmix64": (_U64, [_U64, _U64, _U64]),
        "orc_fill_uniform_f32": (None, [_f32p, ctypes.c_size_t, _U64, _U64, ctypes.c_float, ctypes.c_float]),
        "orc_fill_normal_f32": (None, [_f32p, ctypes.c_size_t, _U64, _U64, ctypes.c_float, ctypes.c_float]),
        "orc_gemm_f64": (None, [ctypes.c_int, ctypes.c_int, _L, _L, _L, ctypes.c_double, _f32p, _L, _f32p, _L,
                                ctypes.c_double, _f64p, _L, ctypes.c_int]),
        "orc_gemm_f64_rows": (None, [ctypes.c_int, ctypes.c_int, _L, _L, _L, _f32p, _L, _f32p, _L, _i64p, _L,
                                     _f64p, _L, ctypes.c_int]),
        "orc_f32_to_f16_rtz": (ctypes.c_uint16, [ctypes.c_float]),
        "orc_f32_to_f16_rne": (ctypes.c_uint16, [ctypes.c_float]),
        "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "orc_cast_f32_f16": (None, [_f32p, _u16p, ctypes.c_size_t, ctypes.c_int]),
        "orc_cast_f16_f32": (None, [_u16p, _f32p, ctypes.c_size_t]),
        "orc_coo_to_csr": (ctypes.c_int, [_L, _L, _L, _i32p, _i32p, _f32p, _i32p, _i32p, _f32p]),
        "orc_csr_to_dense": (None, [_L, _L, _i32p, _i32p, _f32p, _f32p]),
        "orc_spmm_csr_f32": (None, [_L, _L, _i32p, _i32p, _f32p, _f32p, _L, _f32p, _L, ctypes.c_int]),
        "orc_spmm_csr_f64": (None, [_L, _L, _i32p, _i32p, _f32p, _f32p, _L, _f64p, _L, ctypes.c_int]),
        "orc_spmv_csr_f32": (None, [_L, _i32p, _i32p, _f32p, _f32p, _f32p, ctypes.c_int]),
        "orc_spmv_csr_f64": (None, [_L, _i32p, _i32p, _f32p, _f32p, _f64p]),
        "orc_spmm_csr_f32_par": (None, [_L, _L, _i32p, _i32p, _f32p, _f32p, _L, _f32p, _L, ctypes.c_int,
                                        ctypes.c_int]),
        "orc_spmv_csr_f32_par": (None, [_L, _i32p, _i32p, _f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int]),
        "orc_act_f64": (ctypes.c_double, [ctypes.c_int, ctypes.c_double, ctypes.c_double]),
        "orc_softmax_rows_f64": (None, [_L, _L, _f32p, _f64p]),
        "orc_act_f32": (ctypes.c_float, [ctypes.c_int, ctypes.c_float, ctypes.c_float]),
        "orc_spgemm_csr_csc_f32": (None, [_L, _L, _i32p, _i32p, _f32p, _i32p, _i32p, _f32p, _f32p, _L, ctypes.c_int]),
        "orc_dense_csc_f32": (None, [_L, _L, _L, _f32p, _L, _i32p, _i32p, _f32p, _f32p, _L, ctypes.c_int]),
        "orc_sparse_add": (ctypes.c_int, [_L, _i32p, _i32p, _f32p, _i32p, _i32p, _f32p, _i32p, _i32p, _f32p, _L,
                                          ctypes.POINTER(_L)]),
        "orc_dense_to_coo": (ctypes.c_int, [_L, _L, _f32p, ctypes.c_float, _i32p, _i32p, _f32p, _L,
                                            ctypes.POINTER(_L)]),
        "orc_act_grad_f64": (ctypes.c_double, [ctypes.c_int, ctypes.c_double, ctypes.c_double]),
        "orc_act_backward_f64": (None, [ctypes.c_int, ctypes.c_double, ctypes.c_double, _f32p, _f32p, _L, _f64p]),
        "orc_linear_f64": (None, [_L, _L, _L, _f32p, _f32p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                  ctypes.c_double, _f64p, ctypes.c_int]),
        "orc_transpose_f32": (None, [_L, _L, _f32p, _f32p]),
        "orc_act_backward_out_array_f32": (None, [ctypes.c_int, ctypes.c_float, _f32p, _f32p, _f32p, _L]),
        "orc_softmax_backward_f32": (None, [_L, _L, _f32p, _f32p, _f32p]),
        "orc_rel_frob": (ctypes.c_double, [_f32p, _f64p, ctypes.c_size_t]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def threads():
    return max(1, min(16, os.cpu_count() or 1))


# ---------------------------------------------------------------- generators
def uniform(shape, seed, stream, lo=-1.0, hi=1.0):
    out = np.empty(shape, dtype=np.float32)
    lib().orc_fill_uniform_f32(out.reshape(-1), out.size, seed, stream, lo, hi)
    return out


def normal(shape, seed, stream, mean=0.0, std=1.0):
    out = np.empty(shape, dtype=np.float32)
    lib().orc_fill_normal_f32(out.reshape(-1), out.size, seed, stream, mean, std)
    return out


# ---------------------------------------------------------------- GEMM
def _op_dims(X, trans):
    return (X.shape[1], X.shape[0]) if trans else X.shape


def gemm_f64(A, B, transA=False, transB=False, alpha=1.0, beta=0.0, C=None, nthreads=None):
    A = np.ascontiguousarray(A, dtype=np.float32)
    B = np.ascontiguousarray(B, dtype=np.float32)
    M, K = _op_dims(A, transA)
    K2, N = _op_dims(B, transB)
    assert K == K2, (A.shape, B.shape)
    out = np.zeros((M, N), dtype=np.float64) if C is None else np.ascontiguousarray(C, dtype=np.float64).copy()
    lib().orc_gemm_f64(int(transA), int(transB), M, N, K, alpha, A.reshape(-1) if A.size else np.zeros(1, np.float32),
                       A.shape[1] if A.ndim == 2 and A.shape[1] else 1, B.reshape(-1) if B.size else np.zeros(1, np.float32),
                       B.shape[1] if B.ndim == 2 and B.shape[1] else 1, beta, out.reshape(-1) if out.size else np.zeros(1),
                       max(N, 1), nthreads or threads())
    return out


def gemm_f64_rows(A, B, rows, transA=False, transB=False, nthreads=None):
    A = np.ascontiguousarray(A, dtype=np.float32)
    B = np.ascontiguousarray(B, dtype=np.float32)
    M, K = _op_dims(A, transA)
    _, N = _op_dims(B, transB)
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    out = np.zeros((rows.size, N), dtype=np.float64)
    lib().orc_gemm_f64_rows(int(transA), int(transB), M, N, K, A.reshape(-1), A.shape[1], B.reshape(-1),
                            B.shape[1], rows, rows.size, out.reshape(-1), N, nthreads or threads())
    return out


# ---------------------------------------------------------------- fp16
def f32_to_f16_bits(x, rtz):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_cast_f32_f16(x.reshape(-1), out.reshape(-1), x.size, int(bool(rtz)))
    return out


def f16_bits_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_cast_f16_f32(h.reshape(-1), out.reshape(-1), h.size)
    return out


def round_f16(x, rtz):
    """fp32 -> fp16 -> fp32 (the values an fp16 GEMM actually multiplies)."""
    return f16_bits_to_f32(f32_to_f16_bits(x, rtz))


# ---------------------------------------------------------------- sparse
def coo_to_csr(rows, cols, ri, ci, v):
    ri = np.ascontiguousarray(ri, dtype=np.int32)
    ci = np.ascontiguousarray(ci, dtype=np.int32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    nnz = v.size
    rowptr = np.zeros(rows + 1, dtype=np.int32)
    idx = np.zeros(max(nnz, 1), dtype=np.int32)
    data = np.zeros(max(nnz, 1), dtype=np.float32)
    pad = lambda a, dt: a if a.size else np.zeros(1, dt)
    rc = lib().orc_coo_to_csr(rows, cols, nnz, pad(ri, np.int32), pad(ci, np.int32), pad(v, np.float32),
                              rowptr, idx, data)
    return rc, rowptr, idx[:nnz], data[:nnz]


def csr_to_dense(rows, cols, rowptr, idx, data):
    out = np.zeros((rows, cols), dtype=np.float32)
    pad = lambda a, dt: np.ascontiguousarray(a, dtype=dt) if len(a) else np.zeros(1, dt)
    lib().orc_csr_to_dense(rows, cols, np.ascontiguousarray(rowptr, np.int32), pad(idx, np.int32),
                           pad(data, np.float32), out.reshape(-1))
    return out


def spmm_f32(rowptr, col, val, D, use_fma=True):
    M = rowptr.size - 1
    D = np.ascontiguousarray(D, dtype=np.float32)
    N = D.shape[1]
    C = np.empty((M, N), dtype=np.float32)
    pad = lambda a, dt: np.ascontiguousarray(a, dtype=dt) if len(a) else np.zeros(1, dt)
    lib().orc_spmm_csr_f32(M, N, np.ascontiguousarray(rowptr, np.int32), pad(col, np.int32), pad(val, np.float32),
                           D.reshape(-1), N, C.reshape(-1), N, int(use_fma))
    return C


def spmm_f32_par(rowptr, col, val, D, nthreads, use_fma=True):
    """spmm_f32 with the rows split over nthreads OpenMP threads (bit-identical)."""
    M = rowptr.size - 1
    D = np.ascontiguousarray(D, dtype=np.float32)
    N = D.shape[1]
    C = np.empty((M, N), dtype=np.float32)
    lib().orc_spmm_csr_f32_par(M, N, np.ascontiguousarray(rowptr, np.int32), _pad(col, np.int32),
                               _pad(val, np.float32), D.reshape(-1), N, C.reshape(-1), N, int(use_fma), nthreads)
    return C


def spmv_f32_par(rowptr, col, val, x, nthreads, use_fma=True):
    """spmv_f32 with the rows split over nthreads OpenMP threads (bit-identical)."""
    M = rowptr.size - 1
    y = np.empty(max(M, 1), dtype=np.float32)
    lib().orc_spmv_csr_f32_par(M, np.ascontiguousarray(rowptr, np.int32), _pad(col, np.int32), _pad(val, np.float32),
                               _pad(x, np.float32), y, int(use_fma), nthreads)
    return y[:M]


def spmm_f64(rowptr, col, val, D, nthreads=None):
    M = rowptr.size - 1
    D = np.ascontiguousarray(D, dtype=np.float32)
    N = D.shape[1]
    C = np.empty((M, N), dtype=np.float64)
    pad = lambda a, dt: np.ascontiguousarray(a, dtype=dt) if len(a) else np.zeros(1, dt)
    lib().orc_spmm_csr_f64(M, N, np.ascontiguousarray(rowptr, np.int32), pad(col, np.int32), pad(val, np.float32),
                           D.reshape(-1), N, C.reshape(-1), N, nthreads or threads())
    return C


def _pad(a, dt):
    a = np.ascontiguousarray(a, dtype=dt)
    return a if a.size else np.zeros(1, dt)


def spgemm_csr_csc_f32(arp, acol, aval, bcp, brow, bval, use_fma=True):
    """perform_sparse_sparse_matmul restated: A CSR [M, K] x B CSC [K, N] -> dense fp32."""
    M, N = len(arp) - 1, len(bcp) - 1
    C = np.empty((max(M, 1), max(N, 1)), dtype=np.float32)
    lib().orc_spgemm_csr_csc_f32(M, N, _pad(arp, np.int32), _pad(acol, np.int32), _pad(aval, np.float32),
                                 _pad(bcp, np.int32), _pad(brow, np.int32), _pad(bval, np.float32), C.reshape(-1),
                                 C.shape[1], int(use_fma))
    return C[:M, :N]


def dense_csc_f32(A, bcp, brow, bval, use_fma=True):
    """perform_dense_sparse_matmul restated: A dense [M, K] x B CSC [K, N] -> dense fp32."""
    A = np.ascontiguousarray(A, dtype=np.float32)
    M, K = A.shape
    N = len(bcp) - 1
    C = np.empty((max(M, 1), max(N, 1)), dtype=np.float32)
    lib().orc_dense_csc_f32(M, K, N, _pad(A.reshape(-1), np.float32), max(K, 1), _pad(bcp, np.int32),
                            _pad(brow, np.int32), _pad(bval, np.float32), C.reshape(-1), C.shape[1], int(use_fma))
    return C[:M, :N]


def sparse_add(arp, acol, aval, brp, bcol, bval, max_nnz=None):
    """perform_sparse_add restated: returns (rc, rows, cols, vals) of the COO result."""
    M = len(arp) - 1
    cap = len(aval) + len(bval) if max_nnz is None else max_nnz
    ri, ci, vv = np.zeros(max(cap, 1), np.int32), np.zeros(max(cap, 1), np.int32), np.zeros(max(cap, 1), np.float32)
    n = ctypes.c_long(0)
    rc = lib().orc_sparse_add(M, _pad(arp, np.int32), _pad(acol, np.int32), _pad(aval, np.float32),
                              _pad(brp, np.int32), _pad(bcol, np.int32), _pad(bval, np.float32), ri, ci, vv, cap,
                              ctypes.byref(n))
    return rc, ri[:n.value], ci[:n.value], vv[:n.value]


def dense_to_coo(D, threshold, max_nnz=None):
    """perform_dense_to_sparse restated: returns (rc, rows, cols, vals)."""
    D = np.ascontiguousarray(D, dtype=np.float32)
    M, N = D.shape
    cap = M * N if max_nnz is None else max_nnz
    ri, ci, vv = np.zeros(max(cap, 1), np.int32), np.zeros(max(cap, 1), np.int32), np.zeros(max(cap, 1), np.float32)
    n = ctypes.c_long(0)
    rc = lib().orc_dense_to_coo(M, N, _pad(D.reshape(-1), np.float32), threshold, ri, ci, vv, cap, ctypes.byref(n))
    return rc, ri[:n.value], ci[:n.value], vv[:n.value]


def csr_to_csc(rows, cols, rowptr, idx, data):
    """CSR -> CSC by a stable sort on column (ConvertToCSC order, tensor/sparse-tensor.go:184-238):
    returns (colptr, row indices, values)."""
    rowptr = np.asarray(rowptr, np.int64)
    r = np.repeat(np.arange(rows), np.diff(rowptr))
    order = np.lexsort((r, np.asarray(idx)))  # by column, then row
    colptr = np.zeros(cols + 1, np.int32)
    np.cumsum(np.bincount(np.asarray(idx, np.int64), minlength=cols), out=colptr[1:])
    return colptr, r[order].astype(np.int32), np.asarray(data, np.float32)[order]


def spmv_f32(rowptr, col, val, x, use_fma=True):
    M = rowptr.size - 1
    y = np.empty(M, dtype=np.float32)
    pad = lambda a, dt: np.ascontiguousarray(a, dtype=dt) if len(a) else np.zeros(1, dt)
    lib().orc_spmv_csr_f32(M, np.ascontiguousarray(rowptr, np.int32), pad(col, np.int32), pad(val, np.float32),
                           pad(x, np.float32), y if M else np.zeros(1, np.float32), int(use_fma))
    return y


def spmv_f64(rowptr, col, val, x):
    M = rowptr.size - 1
    y = np.empty(max(M, 1), dtype=np.float64)
    pad = lambda a, dt: np.ascontiguousarray(a, dtype=dt) if len(a) else np.zeros(1, dt)
    lib().orc_spmv_csr_f64(M, np.ascontiguousarray(rowptr, np.int32), pad(col, np.int32), pad(val, np.float32),
                           pad(x, np.float32), y)
    return y[:M]


def random_csr(M, K, mean_row, seed, stream=7, distinct=True):
    """Synthetic CSR in the shape of the SpMM workload: row lengths Poisson(mean_row),
    columns uniform and (when distinct) distinct and sorted per row, values U[-1,1]."""
    rng = np.random.default_rng(seed * 1000003 + stream)
    lens = rng.poisson(mean_row, size=M).astype(np.int64)
    lens = np.minimum(lens, K)
    rowptr = np.zeros(M + 1, dtype=np.int64)
    np.cumsum(lens, out=rowptr[1:])
    nnz = int(rowptr[-1])
    col = np.empty(nnz, dtype=np.int32)
    if distinct:
        # sample with replacement, then repair duplicates row by row (rare at 0.1% density)
        raw = rng.integers(0, K, size=nnz, dtype=np.int64)
        for i in range(M):
            s, e = rowptr[i], rowptr[i + 1]
            if e - s == 0:
                continue
            c = np.unique(raw[s:e])
            while c.size < e - s:
                c = np.unique(np.concatenate([c, rng.integers(0, K, size=(e - s) - c.size)]))
            col[s:e] = c
    else:
        col[:] = rng.integers(0, K, size=nnz)
        for i in range(M):
            s, e = rowptr[i], rowptr[i + 1]
            col[s:e].sort()
    val = uniform((nnz,), seed, stream + 1000)
    return rowptr.astype(np.int32), col, val


# ---------------------------------------------------------------- misc
def act_f64(code, x, alpha=0.0):
    f = lib().orc_act_f64
    return np.array([f(code, alpha, float(v)) for v in np.asarray(x, dtype=np.float64).reshape(-1)]).reshape(np.shape(x))


def act_grad_f64(code, x, alpha=0.0):
    """d act / dx at x (orc_act_grad_f64), element-wise, float64."""
    f = lib().orc_act_grad_f64
    return np.array([f(code, alpha, float(v)) for v in np.asarray(x, dtype=np.float64).reshape(-1)]).reshape(np.shape(x))


def act_backward_f64(code, dy, pre, alpha=0.0, scale=1.0):
    """dy * act'(pre) * scale in float64 (orc_act_backward_f64)."""
    dy = np.ascontiguousarray(dy, dtype=np.float32)
    pre = np.ascontiguousarray(pre, dtype=np.float32)
    g = np.empty(pre.shape, dtype=np.float64)
    lib().orc_act_backward_f64(code, alpha, scale, dy.reshape(-1), pre.reshape(-1), pre.size, g.reshape(-1))
    return g


def linear_backward_f64(X, W, pre, dY, act, alpha=0.0, scale=1.0, act_applied=True):
    """Backward of Y = act(X W + b), W [in, out] (FusedLinearActivation.Backward,
    gpu/matrix/fused-operations.go:467-578): returns (dX = G W^T, dW = X^T G,
    db = column sums of G) with G = dY * act'(pre) * scale (G = dY * scale when the
    activation backward is skipped)."""
    G = act_backward_f64(act if act_applied else -1, dY, pre, alpha, scale)
    G32 = G.astype(np.float64)
    dX = G32 @ np.asarray(W, dtype=np.float64).T
    dW = np.asarray(X, dtype=np.float64).T @ G32
    return dX, dW, G32.sum(axis=0), G


def softmax_rows_f64(x):
    """Row-wise softmax of a 2-D fp32 array (a 1-D array is one row) in float64
    (orc_softmax_rows_f64)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    x2 = x.reshape(1, -1) if x.ndim == 1 else x
    out = np.empty(x2.shape, dtype=np.float64)
    lib().orc_softmax_rows_f64(x2.shape[0], x2.shape[1], x2.reshape(-1), out.reshape(-1))
    return out.reshape(x.shape)


def act_f32(code, x, alpha=0.0):
    f = lib().orc_act_f32
    return np.array([f(code, alpha, float(v)) for v in np.asarray(x, dtype=np.float32).reshape(-1)],
                    dtype=np.float32).reshape(np.shape(x))


def linear_f64(X, W, bias, act, w_out_in, alpha=0.0, nthreads=None):
    X = np.ascontiguousarray(X, dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.float32)
    batch, fin = X.shape
    out = W.shape[0] if w_out_in else W.shape[1]
    Y = np.empty((batch, out), dtype=np.float64)
    b = None
    if bias is not None:
        b = np.ascontiguousarray(bias, dtype=np.float32)
    lib().orc_linear_f64(batch, fin, out, X.reshape(-1), W.reshape(-1), int(w_out_in),
                         b.ctypes.data if b is not None else None, act, alpha, Y.reshape(-1), nthreads or threads())
    return Y


def act_backward_out_f32(code, g, y, alpha=0.0):
    """The reference bridge's activation backward from the activation OUTPUT y
    (orc_act_backward_out_f32), element-wise, fp32."""
    g = np.ascontiguousarray(g, dtype=np.float32)
    y = np.ascontiguousarray(y, dtype=np.float32)
    out = np.empty(y.shape, dtype=np.float32)
    lib().orc_act_backward_out_array_f32(code, alpha, g.reshape(-1), y.reshape(-1), out.reshape(-1), y.size)
    return out


def softmax_backward_f32(g, y):
    """y * (g - dot(g, y)) per row (a 1-D array is one row), sequential fp32 dot
    (orc_softmax_backward_f32)."""
    g = np.ascontiguousarray(g, dtype=np.float32)
    y = np.ascontiguousarray(y, dtype=np.float32)
    rows, cols = (1, y.size) if y.ndim == 1 else y.shape
    out = np.empty(y.shape, dtype=np.float32)
    lib().orc_softmax_backward_f32(rows, cols, g.reshape(-1), y.reshape(-1), out.reshape(-1))
    return out


def transpose_f32(X):
    X = np.ascontiguousarray(X, dtype=np.float32)
    out = np.empty((X.shape[1], X.shape[0]), dtype=np.float32)
    lib().orc_transpose_f32(X.shape[0], X.shape[1], X.reshape(-1), out.reshape(-1))
    return out


def rel_frob(X, R):
    X = np.ascontiguousarray(X, dtype=np.float32).reshape(-1)
    R = np.ascontiguousarray(R, dtype=np.float64).reshape(-1)
    return lib().orc_rel_frob(X, R, X.size)
