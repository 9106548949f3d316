"""ctypes binding of libgonngpu.so, the MI355X GEMM / SpMM backend (C ABI in
include/gonngpu.h).

This module only marshals arguments: every computation runs in the HIP library.
If the library is missing, importing works but the first call raises
GonngpuUnavailable; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REPO_DIR = os.path.dirname(PKG_DIR)
LIB_PATH = os.path.join(PKG_DIR, "lib", "libgonngpu.so")
HEADER_PATH = os.path.join(REPO_DIR, "include", "gonngpu.h")

GN_F32, GN_F16 = 0, 1
ROUND_NEAREST_EVEN, ROUND_TOWARD_ZERO = 0, 1
ACT_NONE, ACT_RELU, ACT_SIGMOID, ACT_TANH, ACT_LEAKY_RELU, ACT_ELU, ACT_SWISH, ACT_GELU = -1, 0, 1, 2, 4, 5, 6, 7


class GonngpuUnavailable(RuntimeError):
    pass


class GonngpuError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(f"gonngpu error {code}: {message}")
        self.code = code
        self.message = message


class CError(ctypes.Structure):
    _fields_ = [("message", ctypes.c_void_p)]


_VP = ctypes.c_void_p
_L = ctypes.c_long
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t
_U64 = ctypes.c_uint64
_ERR = ctypes.POINTER(CError)

SIGNATURES = {
    "create_gpu_buffer": (_I, [_VP, _L, ctypes.POINTER(_VP), ctypes.POINTER(_VP), _ERR]),
    "retrieve_gpu_buffer_data": (_I, [_VP, _VP, _L, _ERR]),
    "release_gpu_buffer": (_I, [_VP]),
    "perform_mps_matrix_multiplication": (_I, [_VP, _L, _L, _VP, _L, _L, _VP, _L, _L, _VP, _ERR]),
    "perform_mps_matrix_transpose": (_I, [_VP, _L, _L, _VP, _L, _L, _VP, _ERR]),
    "perform_optimized_gemm": (_I, [_VP, _VP, _VP, _L, _L, _L, _F, _F, _VP, _ERR]),
    "perform_batch_matmul_optimized": (_I, [_VP, _VP, _VP, _L, _L, _L, _L, _VP, _ERR]),
    "perform_fused_linear_activation": (_I, [_VP, _L, _L, _VP, _L, _VP, _I, _F, _VP, _VP, _ERR]),
    "perform_sparse_dense_matmul": (_I, [_VP, _VP, _L, _VP, _L, _L, _L, _L, _VP, _L, _L, _VP, _L, _L, _VP, _ERR]),
    "perform_sparse_matvec": (_I, [_VP, _VP, _L, _VP, _L, _L, _L, _L, _VP, _L, _VP, _L, _VP, _ERR]),
    "perform_sparse_sparse_matmul": (_I, [_VP, _VP, _L, _VP, _L, _L, _L, _L, _VP, _VP, _L, _VP, _L, _L, _L, _L, _VP,
                                          _L, _L, _VP, _ERR]),
    "perform_dense_sparse_matmul": (_I, [_VP, _L, _L, _VP, _VP, _L, _VP, _L, _L, _L, _L, _VP, _L, _L, _VP, _ERR]),
    "perform_sparse_add": (_I, [_VP, _VP, _L, _VP, _L, _L, _L, _L, _VP, _VP, _L, _VP, _L, _L, _L, _L, _VP, _VP, _VP,
                                ctypes.POINTER(_L), _L, _VP, _ERR]),
    "perform_sparse_scalar_multiply": (_I, [_VP, _VP, _L, _VP, _L, _L, _L, _L, _F, _VP, _ERR]),
    "perform_sparse_to_dense": (_I, [_VP, _VP, _L, _VP, _L, _L, _L, _L, _VP, _L, _L, _VP, _ERR]),
    "perform_dense_to_sparse": (_I, [_VP, _L, _L, _F, _VP, _VP, _VP, ctypes.POINTER(_L), _L, _VP, _ERR]),
    "free_c_error_message": (None, [_VP]),
    "gn_version": (ctypes.c_char_p, []),
    "gn_init": (_I, [_ERR]),
    "gn_stream": (_VP, []),
    "gn_buffer_device_ptr": (_VP, [_VP]),
    "gn_buffer_bytes": (_L, [_VP]),
    "gn_memory_stats": (None, [ctypes.POINTER(_L), ctypes.POINTER(_L), ctypes.POINTER(_L)]),
    "gn_malloc": (_I, [ctypes.POINTER(_VP), _SZ, _ERR]),
    "gn_free": (_I, [_VP]),
    "gn_free_async": (_I, [_VP, _VP]),
    "gn_csr_indices_changed": (_I, [_VP]),
    "gn_synchronize": (_I, [_VP, _ERR]),
    "gn_gemm": (_I, [_I, _I, _I, _L, _L, _L, _F, _VP, _L, _L, _VP, _L, _L, _F, _VP, _L, _L, _L, _VP, _I, _F, _VP,
                     _ERR]),
    "gn_cast_f32_f16": (_I, [_VP, _VP, _SZ, _I, _VP, _ERR]),
    "gn_cast_f16_f32": (_I, [_VP, _VP, _SZ, _VP, _ERR]),
    "gn_activation_backward": (_I, [_VP, _VP, _L, _L, _I, _F, _F, _VP, _VP, _VP, _ERR]),
    "gn_activation_backward_noalloc": (_I, [_VP, _VP, _L, _L, _I, _F, _F, _VP, _VP, _VP, _ERR]),
    "gn_transpose_f32": (_I, [_VP, _L, _L, _VP, _VP, _ERR]),
    "gn_activation_forward": (_I, [_VP, _VP, _L, _I, _F, _VP, _ERR]),
    "createMPSGraph": (_VP, []),
    "createMatMulNode": (_VP, [_VP, _VP, _VP]),
    "createReLUNode": (_VP, [_VP, _VP]),
    "compileGraph": (_VP, [_VP, _VP]),
    "executeCompiledGraph": (None, [_VP, _VP, ctypes.POINTER(_VP), _L, ctypes.POINTER(_VP), _L]),
    "gn_graph_placeholder": (_VP, [_VP, _L, _L, _I]),
    "gn_graph_matmul": (_VP, [_VP, _VP, _VP, _I, _I]),
    "gn_graph_activation": (_VP, [_VP, _VP, _I, _F]),
    "gn_graph_compile": (_I, [_VP, ctypes.POINTER(_VP), _L, ctypes.POINTER(_VP), _L, ctypes.POINTER(_VP), _ERR]),
    "gn_graph_execute": (_I, [_VP, _VP, ctypes.POINTER(_VP), _L, ctypes.POINTER(_VP), _L, _ERR]),
    "gn_graph_release": (None, [_VP]),
    "gn_softmax_rows": (_I, [_VP, _VP, _L, _L, _VP, _ERR]),
    "perform_activation_relu_forward": (_I, [_VP, _L, _VP, _VP, _ERR]),
    "perform_activation_sigmoid_forward": (_I, [_VP, _L, _VP, _VP, _ERR]),
    "perform_activation_tanh_forward": (_I, [_VP, _L, _VP, _VP, _ERR]),
    "perform_activation_softmax_1d_forward": (_I, [_VP, _L, _VP, _VP, _ERR]),
    "perform_activation_softmax_2d_forward": (_I, [_VP, _L, _L, _VP, _VP, _ERR]),
    "perform_activation_leaky_relu_forward": (_I, [_VP, _L, _F, _VP, _VP, _ERR]),
    "perform_activation_elu_forward": (_I, [_VP, _L, _F, _VP, _VP, _ERR]),
    "perform_activation_swish_forward": (_I, [_VP, _L, _VP, _VP, _ERR]),
    "perform_activation_gelu_forward": (_I, [_VP, _L, _VP, _VP, _ERR]),
    "gn_spmm_csr": (_I, [_L, _L, _L, _L, _VP, _VP, _VP, _VP, _L, _VP, _L, _VP, _VP, _ERR]),
    "gn_spmv_csr": (_I, [_L, _L, _L, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _ERR]),
    "gn_spmv_plan_create": (_I, [_L, _L, _L, _VP, _VP, ctypes.POINTER(_VP), _VP, _ERR]),
    "gn_spmv_plan_run": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _ERR]),
    "gn_spmv_plan_release": (None, [_VP, _VP]),
    "gn_fill_uniform_f32": (_I, [_VP, _SZ, _U64, _U64, _F, _F, _VP, _ERR]),
    "gn_fill_normal_f32": (_I, [_VP, _SZ, _U64, _U64, _F, _F, _VP, _ERR]),
    # Part 3: the other reference-bridge entries with a device implementation. The rest of
    # Part 3 (entries that report "not provided") has no Python binding.
    "perform_mps_matrix_add": (_I, [_VP, _L, _L, _VP, _L, _L, _VP, _L, _L, _VP, _ERR]),
    "perform_mps_matrix_add_broadcast": (_I, [_VP, _L, _L, _VP, _L, _L, _VP, _L, _L, _VP, _ERR]),
    "perform_mps_matrix_subtract": (_I, [_VP, _L, _L, _VP, _L, _L, _VP, _L, _L, _VP, _ERR]),
    "perform_mps_matrix_element_multiply": (_I, [_VP, _L, _L, _VP, _L, _L, _VP, _L, _L, _VP, _ERR]),
    "perform_mps_matrix_element_divide": (_I, [_VP, _L, _L, _VP, _L, _L, _VP, _L, _L, _VP, _ERR]),
    "perform_mps_matrix_scalar_add": (_I, [_VP, _L, _L, _F, _VP, _VP, _ERR]),
    "perform_mps_matrix_scalar_multiply": (_I, [_VP, _L, _L, _F, _VP, _VP, _ERR]),
    "perform_activation_relu_backward": (_I, [_VP, _VP, _L, _VP, _VP, _ERR]),
    "perform_activation_sigmoid_backward": (_I, [_VP, _VP, _L, _VP, _VP, _ERR]),
    "perform_activation_tanh_backward": (_I, [_VP, _VP, _L, _VP, _VP, _ERR]),
    "perform_activation_softmax_1d_backward": (_I, [_VP, _VP, _L, _VP, _VP, _ERR]),
    "perform_activation_softmax_2d_backward": (_I, [_VP, _VP, _L, _L, _VP, _VP, _ERR]),
    "perform_activation_leaky_relu_backward": (_I, [_VP, _VP, _L, _F, _VP, _VP, _ERR]),
    "perform_activation_elu_backward": (_I, [_VP, _VP, _L, _F, _VP, _VP, _ERR]),
    "perform_activation_swish_backward": (_I, [_VP, _VP, _L, _VP, _VP, _ERR]),
    "perform_activation_gelu_backward": (_I, [_VP, _VP, _L, _VP, _VP, _ERR]),
    "getGPUMemoryUsage": (None, [ctypes.POINTER(_L), ctypes.POINTER(_L)]),
}

_lib = None


def header_symbols(path=HEADER_PATH):
    """Function names declared in include/gonngpu.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b([A-Za-z_][A-Za-z0-9_]*)\s*\(", text, flags=re.M)))


def load(path=LIB_PATH):
    """Loads the library (no device work). Raises GonngpuUnavailable if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise GonngpuUnavailable(f"{path} is not built; run __graft_entry__.build()")
    L = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _check(rc, err):
    if rc != 0:
        msg = ""
        if err.message:
            msg = ctypes.string_at(err.message).decode(errors="replace")
            _lib.free_c_error_message(err.message)
        raise GonngpuError(rc, msg)


def call(name, *args):
    """Calls a C-ABI entry point whose last argument is CError*; raises GonngpuError on failure."""
    L = load()
    err = CError()
    rc = getattr(L, name)(*args, ctypes.byref(err))
    _check(rc, err)
    return rc


def call_rc(name, *args):
    """Like call() but returns (code, message) instead of raising."""
    L = load()
    err = CError()
    rc = getattr(L, name)(*args, ctypes.byref(err))
    msg = ""
    if err.message:
        msg = ctypes.string_at(err.message).decode(errors="replace")
        L.free_c_error_message(err.message)
    return rc, msg


def init():
    call("gn_init")


def stream():
    return load().gn_stream()


def memory_stats():
    cur, peak, n = _L(), _L(), _L()
    load().gn_memory_stats(ctypes.byref(cur), ctypes.byref(peak), ctypes.byref(n))
    return cur.value, peak.value, n.value


# --------------------------------------------------------------------------- GPUPtr handles
class Buffer:
    """A library-owned device buffer (the GPUPtr of the reference bridge)."""

    def __init__(self, nbytes=None, data=None):
        self.handle = _VP()
        dev = _VP()
        if data is not None:
            self._host = np.ascontiguousarray(data)
            nbytes = self._host.nbytes
            src = self._host.ctypes.data_as(_VP)
        else:
            src = None
        call("create_gpu_buffer", src, int(nbytes), ctypes.byref(self.handle), ctypes.byref(dev))
        self.nbytes = int(nbytes)
        self.device = dev.value
        self._host = None

    @classmethod
    def from_array(cls, arr):
        return cls(data=np.ascontiguousarray(arr, dtype=np.float32))

    def to_array(self, shape, dtype=np.float32):
        out = np.empty(shape, dtype=dtype)
        call("retrieve_gpu_buffer_data", self.handle, out.ctypes.data_as(_VP), out.nbytes)
        return out

    @property
    def device_ptr(self):
        return load().gn_buffer_device_ptr(self.handle)

    def release(self):
        if self.handle and self.handle.value:
            load().release_gpu_buffer(self.handle)
            self.handle = _VP()

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


# --------------------------------------------------------------------------- device-pointer API
def _run_ordered(name, *args):
    """Runs a device-pointer entry point ordered with torch's current stream.

    The C ABI takes a stream argument (NULL = the library's own stream). Torch
    tensors are produced on torch's current stream, so the call is issued on that
    stream; if it is the legacy default stream (handle 0), the device is
    synchronized around a call on the library stream instead."""
    import torch

    sp = torch.cuda.current_stream().cuda_stream
    if sp:
        return call(name, *args, sp)
    torch.cuda.synchronize()
    call(name, *args, None)
    call("gn_synchronize", None)


def _ptr(t):
    """Device address of a torch tensor / int / None."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def gemm(A, B, C, *, transA=False, transB=False, alpha=1.0, beta=0.0, bias=None, act=ACT_NONE, act_alpha=0.0,
         M=None, N=None, K=None, lda=None, ldb=None, ldc=None, batch=1, strideA=0, strideB=0, strideC=0,
         dtype=None, stream_ptr=None):
    """C = act(alpha*op(A)*op(B) + beta*C + bias) on torch device tensors (row-major, last two dims)."""
    import torch

    if dtype is None:
        dtype = GN_F16 if A.dtype == torch.float16 else GN_F32
    a_rows, a_cols = A.shape[-2], A.shape[-1]
    b_rows, b_cols = B.shape[-2], B.shape[-1]
    M = M if M is not None else (a_cols if transA else a_rows)
    K = K if K is not None else (a_rows if transA else a_cols)
    N = N if N is not None else (b_rows if transB else b_cols)
    lda = lda if lda is not None else A.stride(-2)
    ldb = ldb if ldb is not None else B.stride(-2)
    ldc = ldc if ldc is not None else C.stride(-2)
    _dispatch(stream_ptr, "gn_gemm", dtype, int(transA), int(transB), M, N, K, alpha, _ptr(A), lda, strideA, _ptr(B),
              ldb, strideB, beta, _ptr(C), ldc, strideC, batch, _ptr(bias), act, act_alpha)


def cast_f32_f16(x, out, round_mode=ROUND_NEAREST_EVEN, stream_ptr=None):
    _dispatch(stream_ptr, "gn_cast_f32_f16", _ptr(x), _ptr(out), x.numel(), round_mode)


def cast_f16_f32(x, out, stream_ptr=None):
    _dispatch(stream_ptr, "gn_cast_f16_f32", _ptr(x), _ptr(out), x.numel())


def activation_backward(grad_out, pre, act, grad_in, grad_bias=None, alpha=0.0, scale=1.0, stream_ptr=None):
    """grad_in = grad_out * act'(pre) * scale; grad_bias = column sums of grad_in (optional)."""
    rows, cols = pre.shape
    _dispatch(stream_ptr, "gn_activation_backward", _ptr(grad_out), _ptr(pre), rows, cols, act, alpha, scale,
              _ptr(grad_in), _ptr(grad_bias))


def activation_forward(x, out, act, alpha=0.0, stream_ptr=None):
    """out = act(x) element-wise (ActivationType code other than Softmax, or ACT_NONE)."""
    _dispatch(stream_ptr, "gn_activation_forward", _ptr(x), _ptr(out), x.numel(), act, alpha)


def softmax_rows(x, out, stream_ptr=None):
    """Row-wise softmax of a 2-D tensor (a 1-D tensor is one row)."""
    rows, cols = (1, x.shape[0]) if x.dim() == 1 else (x.shape[0], x.shape[1])
    _dispatch(stream_ptr, "gn_softmax_rows", _ptr(x), _ptr(out), rows, cols)


def transpose(x, out, stream_ptr=None):
    _dispatch(stream_ptr, "gn_transpose_f32", _ptr(x), x.shape[0], x.shape[1], _ptr(out))


def spmm_csr(M, N, K, nnz, rowptr, col, val, D, C, flags=None, ldd=None, ldc=None, stream_ptr=None):
    _dispatch(stream_ptr, "gn_spmm_csr", M, N, K, nnz, _ptr(rowptr), _ptr(col), _ptr(val), _ptr(D),
              ldd if ldd is not None else N, _ptr(C), ldc if ldc is not None else N, _ptr(flags))


def spmv_csr(M, K, nnz, rowptr, col, val, x, y, flags=None, stream_ptr=None):
    _dispatch(stream_ptr, "gn_spmv_csr", M, K, nnz, _ptr(rowptr), _ptr(col), _ptr(val), _ptr(x), _ptr(y), _ptr(flags))


class SpmvPlan:
    """A grouped-layout SpMV plan over device CSR arrays (gn_spmv_plan_*). The row pointer
    and column tensors must outlive the plan and stay unchanged."""

    def __init__(self, M, K, nnz, rowptr, col, stream_ptr=None):
        import torch

        self.handle = _VP()
        self._keep = (rowptr, col)
        sp = stream_ptr if stream_ptr is not None else torch.cuda.current_stream().cuda_stream
        call("gn_spmv_plan_create", M, K, nnz, _ptr(rowptr), _ptr(col), ctypes.byref(self.handle), sp or None)
        self._stream = sp or None

    def run(self, val, x, y, flags=None, stream_ptr=None):
        _dispatch(stream_ptr, "gn_spmv_plan_run", self.handle, _ptr(val), _ptr(x), _ptr(y), _ptr(flags))

    def release(self, stream_ptr=None):
        if self.handle:
            load().gn_spmv_plan_release(self.handle, stream_ptr if stream_ptr is not None else self._stream)
            self.handle = _VP()


def fill_uniform(out, seed, stream_id, lo=-1.0, hi=1.0, stream_ptr=None):
    _dispatch(stream_ptr, "gn_fill_uniform_f32", _ptr(out), out.numel(), seed, stream_id, lo, hi)


def fill_normal(out, seed, stream_id, mean=0.0, std=1.0, stream_ptr=None):
    _dispatch(stream_ptr, "gn_fill_normal_f32", _ptr(out), out.numel(), seed, stream_id, mean, std)


def synchronize(stream_ptr=None):
    call("gn_synchronize", stream_ptr)


def _dispatch(stream_ptr, name, *args):
    """Explicit stream -> call on it; otherwise order with torch's current stream."""
    if stream_ptr is not None:
        return call(name, *args, stream_ptr)
    return _run_ordered(name, *args)
