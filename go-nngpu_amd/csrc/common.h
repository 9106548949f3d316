// common.h — internal declarations shared by the HIP translation units of
// libgonngpu.so (runtime, kernels, C-ABI bridge). Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <mutex>

#include "../../include/gonngpu.h"

namespace gn {

// ---------------------------------------------------------------- errors
// Formats into a malloc'd message stored in err (if non-NULL) and returns code.
int set_error(CError *err, int code, const char *fmt, ...) __attribute__((format(printf, 3, 4)));
// Maps a failed HIP call to code with "<what>: <hip error string>".
int hip_error(CError *err, int code, const char *what, hipError_t e);

// Bytes of a rows x cols matrix of esz-byte elements in *out; false when a size is
// negative or the product overflows (caller-supplied sizes must not wrap into a small
// allocation or a passing bounds check).
inline bool matrix_bytes(long rows, long cols, size_t esz, size_t *out) {
  if (rows < 0 || cols < 0) return false;
  size_t n;
  return !__builtin_mul_overflow((size_t)rows, (size_t)cols, &n) && !__builtin_mul_overflow(n, esz, out);
}

// ---------------------------------------------------------------- context
struct Context {
  int device = 0;
  hipStream_t stream = nullptr;
  int num_cus = 0;
  size_t lds_per_block = 0;
  char arch[64] = {0};
};
// Initialises the process-wide context once; returns nullptr (and sets err) on failure.
Context *context(CError *err);
hipStream_t resolve_stream(void *stream);  // NULL -> library stream

// ---------------------------------------------------------------- allocator
// Caching device allocator: size-binned free lists over hipMalloc, never returns
// memory to the driver while the process lives (reuse keeps hipMalloc off hot paths).
// Release is stream-ordered: dev_free_on(p, s) hands p to a new owner only after the
// work enqueued on s before the call has completed; dev_free orders on the library
// stream (every Part-1 call and every scratch block of the library runs there).
void *dev_alloc(size_t bytes, CError *err);
void dev_free_on(void *p, hipStream_t s);
void dev_free(void *p);
void memory_stats(long *cur, long *peak, long *n);
// Device scratch owned by the library, one block per stream, grown on demand (the old
// block is released in the stream's order). lk holds a library mutex on return: keep it until every
// kernel that uses the scratch is enqueued, so that another host thread cannot enqueue
// work that reuses it in between (kernels on one stream run in order).
void *stream_scratch(hipStream_t s, size_t bytes, std::unique_lock<std::mutex> &lk, CError *err);
// Called with lk still held, after the kernels that use the scratch are enqueued: a block
// above 256 MiB is released (stream-ordered) instead of being kept for the stream's next
// call, so one large call does not pin it for the life of the process.
void stream_scratch_trim(hipStream_t s, std::unique_lock<std::mutex> &lk);

// ---------------------------------------------------------------- host <-> device
// Synchronous copies of pageable host memory through a pinned staging ring.
int upload(void *dst_dev, const void *src_host, size_t bytes, hipStream_t s, CError *err);
int download(void *dst_host, const void *src_dev, size_t bytes, hipStream_t s, CError *err);

// ---------------------------------------------------------------- GPUPtr handles
struct Buffer {
  uint64_t magic;
  void *dptr;
  size_t bytes;
};
constexpr uint64_t kBufferMagic = 0x676E6E6770754246ULL;  // "gnngpuBF"
Buffer *as_buffer(GPUPtr p);  // nullptr if p is not a live handle
// Drops the device copy of the CSR index arrays kept with values buffer b (bridge.cpp).
void csr_cache_drop(const Buffer *b);

// ---------------------------------------------------------------- kernel launchers
// All launchers validate shapes on the host before any launch, then enqueue on s.
struct GemmDesc {
  int dtype;  // GN_F32 / GN_F16
  bool ta, tb;
  long M, N, K;
  float alpha, beta;
  const void *A;
  long lda, strideA;
  const void *B;
  long ldb, strideB;
  float *C;
  long ldc, strideC;
  long batch;
  const float *bias;
  int act;
  float act_alpha;
};
int launch_gemm(const GemmDesc &d, hipStream_t s, CError *err);
int launch_cast_f32_f16(const float *in, uint16_t *out, size_t n, int mode, hipStream_t s, CError *err);
int launch_cast_f16_f32(const uint16_t *in, float *out, size_t n, hipStream_t s, CError *err);
int launch_transpose_f32(const float *in, long rows, long cols, float *out, hipStream_t s, CError *err);
// grad_in = grad_out * act'(pre) * scale element-wise (derivative with respect to the
// pre-activation), and optionally grad_bias[j] = sum over rows of grad_in[., j].
// y = act(x) element-wise over n floats (act.h codes, GN_ACT_NONE copies).
bool act_forward_supported(int act);
int launch_act_forward(const float *in, float *out, long n, int act, float alpha, hipStream_t s, CError *err);
// Row-wise softmax of a row-major [rows, cols] matrix.
int launch_softmax_rows(const float *in, float *out, long rows, long cols, hipStream_t s, CError *err);
int launch_act_backward(const float *grad_out, const float *pre, long rows, long cols, int act, float alpha,
                        float scale, float *grad_in, float *grad_bias, hipStream_t s, CError *err);
// The same computation with the partial column sums in the file-scope `scratch` array of
// elementwise.hip (no allocation on any call); rejects shapes whose partials exceed it.
int launch_act_backward_noalloc(const float *grad_out, const float *pre, long rows, long cols, int act, float alpha,
                                float scale, float *grad_in, float *grad_bias, hipStream_t s, CError *err);
// Looks up the address of that array on the current device (once per device); 0 on success.
int noalloc_scratch_setup(CError *err);
bool act_grad_supported(int act);
int launch_spmm(long M, long N, long K, long nnz, const int32_t *rowptr, const int32_t *col, const float *val,
                const float *D, long ldd, float *C, long ldc, int *flags, hipStream_t s, CError *err);
int launch_spmv(long M, long K, long nnz, const int32_t *rowptr, const int32_t *col, const float *val,
                const float *x, float *y, int *flags, hipStream_t s, CError *err);
int launch_fill_uniform(float *out, size_t n, uint64_t seed, uint64_t sid, float lo, float hi, hipStream_t s,
                        CError *err);
int launch_fill_normal(float *out, size_t n, uint64_t seed, uint64_t sid, float mean, float sd, hipStream_t s,
                       CError *err);
int launch_zero_i32(int *p, long n, hipStream_t s, CError *err);
// sparse_ops.hip (flags as launch_spmm: [0] bad row/column pointers, [1] index out of range)
int launch_spgemm_csr_csc(long M, long N, long annz, long bnnz, const int32_t *arp, const int32_t *acol,
                          const float *aval, const int32_t *bcp, const int32_t *brow, const float *bval, float *C,
                          long ldc, int *flags, hipStream_t s, CError *err);
int launch_spadd(bool write, long M, long N, long annz, long bnnz, const int32_t *arp, const int32_t *acol,
                 const float *aval, const int32_t *brp, const int32_t *bcol, const float *bval, long *count,
                 const long *out_off, int32_t *ri, int32_t *ci, float *vv, int *flags, hipStream_t s, CError *err);
int launch_scale_f32(float *v, long n, float scalar, hipStream_t s, CError *err);
int launch_csr_to_dense(long M, long N, long nnz, const int32_t *rp, const int32_t *col, const float *val, float *D,
                        int *flags, hipStream_t s, CError *err);
int launch_dense_to_coo(bool write, long M, long N, const float *D, float thr, long *count, const long *out_off,
                        int32_t *ri, int32_t *ci, float *vv, hipStream_t s, CError *err);

bool act_supported(int act);

// compat_ops.hip: the element-wise matrix operations and activation backwards of the
// reference bridge. op: 0 add, 1 subtract, 2 multiply, 3 divide; for division
// *first_zero receives the lowest index with b == 0 (-1 when none), which waits for the
// kernel.
int launch_binary_f32(int op, const float *a, const float *b, float *c, long n, long *first_zero, hipStream_t s,
                      CError *err);
// c[i, j] = a[i * sa_r + j * sa_c] + b[i * sb_r + j * sb_c] over an M x N result.
// y[i] += b[i % L], i < n (L > 0).
int launch_add_cyclic_f32(float *y, long n, const float *b, long L, hipStream_t s, CError *err);
int launch_add_broadcast_f32(const float *a, long sa_r, long sa_c, const float *b, long sb_r, long sb_c, float *c,
                             long M, long N, hipStream_t s, CError *err);
// out = in * scalar (mul) or in + scalar.
int launch_scalar_f32(bool mul, const float *in, float scalar, float *out, long n, hipStream_t s, CError *err);
// gin = gradient through an activation, computed from its OUTPUT y (reference formulas).
int launch_act_backward_from_output(const float *gout, const float *y, float *gin, long n, int act, float alpha,
                                    hipStream_t s, CError *err);
// gin = y * (g - dot(g, y)) per row of a [rows, cols] matrix.
int launch_softmax_backward(const float *g, const float *y, float *gin, long rows, long cols, hipStream_t s,
                            CError *err);

// spmv_grouped.hip: CSR SpMV over a one-time layout of the structure (row blocks, entries
// of each block grouped by the 128-byte line of x they gather). Bit-identical to an fmaf
// loop over each row in CSR order.
struct SpmvLayout {
  long M = 0, K = 0, nnz = 0;
  int nblocks = 0, cap = 0;     // blocks (workgroups) and the most entries in one
  int32_t *blk = nullptr;       // nblocks + 1 row starts, then nblocks + 1 entry offsets
  uint32_t *word = nullptr;     // K <= 65536: column | CSR position << 16 | bad-column bit 31
  int32_t *scol = nullptr;      // K > 65536: columns, grouped within each block
  uint16_t *spos = nullptr;     //   and each one's position in its block's CSR order
};
bool spmv_grouped_supported(long M, long K, long nnz);
// Builds the layout for rows [0, M) of a CSR structure whose row pointers are validated
// (non-decreasing within [0, nnz]; host copy h_rowptr) and whose columns are on the device
// (d_col): allocates from the pool and enqueues the grouping kernel on s. Returns 0 when
// built, 1 when the structure does not take the layout (an unsupported shape, or a row of
// more than 4096 entries; *out stays empty), a negative code on failure.
int build_spmv_layout(long M, long K, long nnz, const int32_t *h_rowptr, const int32_t *d_col, int num_cus,
                      hipStream_t s, SpmvLayout *out, CError *err);
void free_spmv_layout(SpmvLayout *l, hipStream_t s);  // stream-ordered on s
// y = S x with the layout; d_rowptr are the structure's row pointers; flags[1] is raised for
// a column outside [0, K).
int launch_spmv_grouped(const SpmvLayout &l, const int32_t *d_rowptr, const float *val, const float *x, float *y,
                        int *flags, hipStream_t s, CError *err);

// bridge.cpp helpers shared with bridge_compat.cpp.
// Waits for the work enqueued on s, as the reference's waitUntilCompleted does; returns
// code (with the HIP error in err) on a device error.
int sync_stream(hipStream_t s, CError *err, int code);
// True when buffer b holds a rows x cols matrix of esz-byte elements.
bool buffer_fits(const Buffer *b, long rows, long cols, size_t esz);

}  // namespace gn

namespace gn {
Buffer *register_buffer(void *dptr, size_t bytes);
bool unregister_buffer(Buffer *b);
}  // namespace gn
