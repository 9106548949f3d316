/*
 * gonngpu.h — C ABI of the MI355X (gfx950) GEMM / SpMM backend for go-nngpu
 * (module github.com/tsawler/gometal).
 *
 * Part 1 re-exports, with identical names and signatures, the subset of the
 * reference bridge header internal/cgo/metal_bridge.h that the matmul path binds
 * (each declaration cites the prototype it replaces): the calls of
 * tensor/tensor.go:130,171,198; gpu/matrix/matrix.go:87,387;
 * gpu/matrix/sparse-matrix.go:167,562; gpu/matrix/optimized-kernels.go:57,118;
 * gpu/matrix/fused-operations.go:441.
 *
 * Part 2 adds gn_* entry points that take raw device pointers, explicit
 * transposes, dtypes, epilogues and a HIP stream; they have no reference
 * counterpart and are what a caller that keeps data resident in HBM uses.
 *
 * Part 3 declares, with the reference prototypes, every other metal_bridge.h function
 * that the Go packages gpu/matrix, gpu/optimizer and tensor call, so that with their
 * cgo preambles pointed at this header and library (and nothing else changed in their
 * code) they compile and link. The element-wise matrix operations and the activation
 * backwards run on the device; the entries of subsystems outside this backend
 * (convolution, losses, optimizers, decompositions, ...) return -1 with a message.
 *
 * Conventions shared by every entry point:
 *  - return 0 on success, a negative code on failure; on failure, if err is
 *    non-NULL, err->message holds a malloc'd string the caller releases with
 *    free_c_error_message() (metal_bridge_common.m:20-34 convention);
 *  - Part-1 calls are synchronous: they return after the device work finished
 *    (as the reference's commit + waitUntilCompleted, metal_bridge_matrix.m:115-116);
 *  - Part-2 calls are asynchronous on the given stream (NULL = the library stream);
 *  - all matrices are row-major; fp32 = IEEE binary32, fp16 = IEEE binary16.
 */
#ifndef GONNGPU_H
#define GONNGPU_H

#include <stddef.h>
#include <stdint.h>
#ifndef __cplusplus
#include <stdbool.h>
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* ========================================================================== */
/* Part 1 — drop-in subset of internal/cgo/metal_bridge.h                      */
/* ========================================================================== */

/* metal_bridge.h:9-11. GPUPtr is an opaque handle to a device buffer owned by this
 * library (HBM allocation + size); DevicePtr is an opaque, non-NULL context token.
 * Callers never dereference either. */
typedef void *GPUPtr;
typedef void *DevicePtr;

/* metal_bridge.h:14-16. */
typedef struct {
  char *message;
} CError;

/* metal_bridge.h:23. Allocates length_bytes of HBM and copies length_bytes from
 * data (host) into it (data may be NULL: the buffer is zero-filled). Unlike the
 * reference (newBufferWithBytesNoCopy, metal_bridge_buffer.m:46-49) the buffer does
 * not alias host memory: later host writes need a new upload.
 * Codes: -1 device unavailable, -3 allocation failed, -4 copy failed. */
int create_gpu_buffer(float *data, long length_bytes, GPUPtr *outGPUPtr, DevicePtr *outDevicePtr, CError *err);

/* metal_bridge.h:24. Copies length_bytes from the buffer into data.
 * Codes: -1 invalid handle, -2 length_bytes exceeds the buffer
 * (metal_bridge_buffer.m:65-72), -4 copy failed. */
int retrieve_gpu_buffer_data(GPUPtr gpuPtr, float *data, long length_bytes, CError *err);

/* metal_bridge.h:25. Returns the allocation to the library's pool, stream-ordered on the
 * library stream (see gn_free_async): it does not wait, and the memory is reused only after
 * the library stream's work enqueued so far (every Part-1 call runs there). NULL is a no-op. */
int release_gpu_buffer(GPUPtr gpuPtr);

/* metal_bridge.h:28-34. C[resultRows,resultCols] = A[aRows,aCols] * B[bRows,bCols],
 * fp32, row-major (metal_bridge_matrix.m:67-97). mtlDevicePtr may be NULL (the
 * reference required a device that its Go caller never set).
 * Codes: -2 NULL buffer, -3 inconsistent dimensions or buffer too small,
 * -6 device execution error. */
int perform_mps_matrix_multiplication(GPUPtr aMatrixPtr, long aRows, long aCols, GPUPtr bMatrixPtr, long bRows,
                                      long bCols, GPUPtr resultMatrixPtr, long resultRows, long resultCols,
                                      DevicePtr mtlDevicePtr, CError *err);

/* metal_bridge.h:36-41. out[j,i] = in[i,j] (metal_bridge_matrix.m:162-166).
 * Codes: -2 dimensions not transposed (:145-148), -3 NULL buffer / too small,
 * -6 device execution error. */
int perform_mps_matrix_transpose(GPUPtr inputMatrixPtr, long inputRows, long inputCols, GPUPtr outputMatrixPtr,
                                 long outputRows, long outputCols, DevicePtr mtlDevicePtr, CError *err);

/* metal_bridge.h:1423-1429. C = alpha*A[M,K]*B[K,N] + beta*C (metal_bridge_kernels.m:81).
 * Codes: -2 NULL buffer, -3 bad sizes / buffer too small, -4 execution error. */
int perform_optimized_gemm(GPUPtr aPtr, GPUPtr bPtr, GPUPtr cPtr, long M, long N, long K, float alpha, float beta,
                           DevicePtr mtlDevicePtr, CError *err);

/* metal_bridge.h:1432-1437. C_b = A_b[M,K]*B_b[K,N] for b < batchSize, batches packed
 * back to back (metal_bridge_kernels.m:85-110). Codes as perform_optimized_gemm. */
int perform_batch_matmul_optimized(GPUPtr aPtr, GPUPtr bPtr, GPUPtr cPtr, long batchSize, long M, long N, long K,
                                   DevicePtr mtlDevicePtr, CError *err);

/* metal_bridge.h:1348-1353. output[b,o] = act(sum_i input[b,i]*weight[i,o] + bias[o]);
 * weight is [input_size, output_size] (fused-operations.go:413-415,
 * default.metal:477-484); bias may be NULL. activation_type uses the Go
 * ActivationType codes (gpu/matrix/activation.go:20-29): 0 ReLU, 1 Sigmoid, 2 Tanh,
 * 4 LeakyReLU(alpha), 5 ELU(alpha), 6 Swish, 7 GELU (tanh form); any other code
 * (including 3 Softmax, which is not element-wise) is rejected with -1.
 * The reference is not consistent about these codes. Its Go caller sends the
 * ActivationType of a non-nil config (fused-operations.go:436-439) but C.int(OpReLU) = 6
 * (the OpType enum, gradient.go:27-39) for a nil one, commented "Default to ReLU" (:433);
 * its kernel reads 0 ReLU, 1 LeakyReLU, 2 Sigmoid, 3 Tanh, 4 GELU and any other code as
 * no activation (default.metal:488-506), so a nil activation would give the plain linear
 * output, had the kernel ever loaded (its library load fails in cgo builds and the call
 * copies the input instead, metal_bridge_fused.m:154-161). This library reads every code
 * as an ActivationType, so code 6 is Swish, and the unchanged Go call with a nil activation
 * runs Swish. The integration changes that one Go line to send ReLU (0), the comment's
 * intent: a deliberate deviation from the kernel's reading (identity).
 * Codes: -1 invalid argument / NULL buffer / execution error (as the reference). */
int perform_fused_linear_activation(GPUPtr input, long batch_size, long input_size, GPUPtr weight, long output_size,
                                    GPUPtr bias, int activation_type, float alpha, GPUPtr output, DevicePtr device,
                                    CError *error);

/* metal_bridge.h:180-187. C = S*B with S in CSR (values in aValuesPtr, host row
 * pointers and column indices valid for the call, sparse-matrix.go:167-177) and B,
 * C dense row-major fp32. Sums duplicates and keeps explicit zeros exactly as the
 * reference loop (metal_bridge_sparse.m:117-133); nnz = 0 returns C = 0.
 * Index residency: the device copy of the index arrays is kept with the values
 * buffer. The first call uploads and validates them; later calls with the same
 * values buffer, the same host arrays and equal row pointers reuse that copy (no
 * upload, no validation read-back). The copy goes with release_gpu_buffer of the
 * values buffer. Column indices changed in place while the values buffer lives need
 * gn_csr_indices_changed(aValuesPtr) before the next call, as changed values need a
 * new upload. The same holds for perform_sparse_matvec, perform_sparse_to_dense and
 * the CSC arrays of perform_dense_sparse_matmul. GONNGPU_CSR_CACHE=0 disables it.
 * Codes: -1 NULL buffer, -2 inconsistent dimensions, -3 malformed CSR
 * (row pointers not monotone / out of [0,nnz], column index outside [0,aCols)),
 * -6 execution error. */
int perform_sparse_dense_matmul(GPUPtr aValuesPtr, int *aRowPtr, long aRowPtrLen, int *aColIndices,
                                long aColIndicesLen, long aRows, long aCols, long aNNZ, GPUPtr bMatrixPtr,
                                long bRows, long bCols, GPUPtr resultMatrixPtr, long resultRows, long resultCols,
                                DevicePtr mtlDevicePtr, CError *err);

/* metal_bridge.h:221-228. y = S*x (metal_bridge_sparse.m:297-342).
 * Codes: -1 dimension mismatch (:306-309) or NULL buffer, -3 malformed CSR,
 * -6 execution error. */
int perform_sparse_matvec(GPUPtr aValuesPtr, int *aRowPtr, long aRowPtrLen, int *aColIndices, long aColIndicesLen,
                          long aRows, long aCols, long aNNZ, GPUPtr xVectorPtr, long xSize, GPUPtr resultVectorPtr,
                          long resultSize, DevicePtr mtlDevicePtr, CError *err);

/* metal_bridge.h:168-176. C = A*B, A in CSR (host row pointers / column indices),
 * B in CSC (host column pointers / row indices), C dense row-major fp32
 * (sparseSparseMatMul, sparse-matrix.go:69-131). Every output runs the reference's
 * merge of A's row with B's column (metal_bridge_sparse.m:56-84): equal indices pair
 * up and both advance, one fma per match; a zero sum stores +0. Either nnz may be 0.
 * Codes: -1 NULL buffer, -2 inconsistent dimensions, -3 malformed row/column
 * pointers, -6 execution error. */
int perform_sparse_sparse_matmul(GPUPtr aValuesPtr, int *aRowPtr, long aRowPtrLen, int *aColIndices,
                                 long aColIndicesLen, long aRows, long aCols, long aNNZ, GPUPtr bValuesPtr,
                                 int *bColPtr, long bColPtrLen, int *bRowIndices, long bRowIndicesLen, long bRows,
                                 long bCols, long bNNZ, GPUPtr resultMatrixPtr, long resultRows, long resultCols,
                                 DevicePtr mtlDevicePtr, CError *err);

/* metal_bridge.h:189-197. C = A*B, A dense row-major, B in CSC (denseSparseMatMul,
 * sparse-matrix.go:193-250). Each output accumulates over B's column entries in
 * order with one fma each (metal_bridge_sparse.m:163-176).
 * Codes: -1 NULL buffer, -2 inconsistent dimensions, -3 malformed CSC (column
 * pointers, or a row index outside [0, bRows)), -6 execution error. */
int perform_dense_sparse_matmul(GPUPtr aMatrixPtr, long aRows, long aCols, GPUPtr bValuesPtr, int *bColPtr,
                                long bColPtrLen, int *bRowIndices, long bRowIndicesLen, long bRows, long bCols,
                                long bNNZ, GPUPtr resultMatrixPtr, long resultRows, long resultCols,
                                DevicePtr mtlDevicePtr, CError *err);

/* metal_bridge.h:199-209. A + B for two CSR matrices into host COO arrays
 * (SparseAdd, sparse-matrix.go:252-320): the reference's per-row merge
 * (metal_bridge_sparse.m:221-259); coinciding entries are added and dropped when the
 * sum is 0, the others are kept as they are. *actualNNZ receives the entry count.
 * Codes: -1 dimension mismatch (:196-199), NULL buffer or bad arguments, -2 more
 * than maxResultNNZ entries (the arrays' contents are then unspecified), -3
 * malformed CSR (including a column index outside [0, aCols)), -6 execution error. */
int perform_sparse_add(GPUPtr aValuesPtr, int *aRowPtr, long aRowPtrLen, int *aColIndices, long aColIndicesLen,
                       long aRows, long aCols, long aNNZ, GPUPtr bValuesPtr, int *bRowPtr, long bRowPtrLen,
                       int *bColIndices, long bColIndicesLen, long bRows, long bCols, long bNNZ,
                       int *resultRowIndices, int *resultColIndices, float *resultValues, long *actualNNZ,
                       long maxResultNNZ, DevicePtr mtlDevicePtr, CError *err);

/* metal_bridge.h:211-218. values[0..nnz) *= scalar in place (SparseScalarMul,
 * sparse-matrix.go:322-364; metal_bridge_sparse.m:286-289). The index arrays are not
 * read. Codes: -1 NULL or too small buffer, -6 execution error. */
int perform_sparse_scalar_multiply(GPUPtr valuesPtr, int *rowPtr, long rowPtrLen, int *colIndices,
                                   long colIndicesLen, long rows, long cols, long nnz, float scalar,
                                   DevicePtr mtlDevicePtr, CError *err);

/* metal_bridge.h:230-236. Dense = CSR (SparseToDense, sparse-matrix.go:425-473):
 * zeros, then each row's entries in CSR order, so a later duplicate overwrites an
 * earlier one (metal_bridge_sparse.m:366-377). Codes: -1 dimension mismatch
 * (:353-356), NULL buffer or bad arrays, -3 malformed CSR (including a column index
 * outside [0, cols)), -6 execution error. */
int perform_sparse_to_dense(GPUPtr valuesPtr, int *rowPtr, long rowPtrLen, int *colIndices, long colIndicesLen,
                            long rows, long cols, long nnz, GPUPtr denseMatrixPtr, long denseRows, long denseCols,
                            DevicePtr mtlDevicePtr, CError *err);

/* metal_bridge.h:239-246. COO of the entries with |v| > threshold, in row-major order,
 * into host arrays (DenseToSparse, sparse-matrix.go:475-525; metal_bridge_sparse.m:
 * 405-424; NaN is never kept). Codes: -1 NULL buffer or bad arguments, -2 more than
 * maxNNZ entries (contents then unspecified), -6 execution error. */
int perform_dense_to_sparse(GPUPtr denseMatrixPtr, long rows, long cols, float threshold, int *rowIndices,
                            int *colIndices, float *values, long *actualNNZ, long maxNNZ, DevicePtr mtlDevicePtr,
                            CError *err);

/* metal_bridge.h:257-396, the forward half (ActivationForward, gpu/matrix/activation.go:
 * 56-175). output = act(input) element-wise over `size` floats, with the reference's
 * formulas (metal_bridge_activation.m): ReLU max(0,x) (:26-51); Sigmoid and Tanh of x
 * clamped to [-88, 88] (:84-110, :145-171); Leaky ReLU x > 0 ? x : alpha*x (:371-397);
 * ELU x > 0 ? x : alpha*(exp(max(x,-88)) - 1) (:435-467); Swish c*sigmoid(c) with
 * c = x clamped to [-88, 88] (:514-542); GELU tanh form, inner argument clamped to
 * [-88, 88] (:606-639). Softmax 1-D over `size` values and 2-D row-wise over
 * [batchSize, features] (:206-242, :283-325): max-subtracted exp, divided by the sum.
 * Input and output may be the same buffer. Codes: -1 NULL or too small buffer,
 * negative size, or execution error (the reference returns -1 for bad buffers). */
int perform_activation_relu_forward(GPUPtr inputPtr, long size, GPUPtr outputPtr, DevicePtr mtlDevicePtr,
                                    CError *err);
int perform_activation_sigmoid_forward(GPUPtr inputPtr, long size, GPUPtr outputPtr, DevicePtr mtlDevicePtr,
                                       CError *err);
int perform_activation_tanh_forward(GPUPtr inputPtr, long size, GPUPtr outputPtr, DevicePtr mtlDevicePtr,
                                    CError *err);
int perform_activation_softmax_1d_forward(GPUPtr inputPtr, long size, GPUPtr outputPtr, DevicePtr mtlDevicePtr,
                                          CError *err);
int perform_activation_softmax_2d_forward(GPUPtr inputPtr, long batchSize, long features, GPUPtr outputPtr,
                                          DevicePtr mtlDevicePtr, CError *err);
int perform_activation_leaky_relu_forward(GPUPtr inputPtr, long size, float alpha, GPUPtr outputPtr,
                                          DevicePtr mtlDevicePtr, CError *err);
int perform_activation_elu_forward(GPUPtr inputPtr, long size, float alpha, GPUPtr outputPtr,
                                   DevicePtr mtlDevicePtr, CError *err);
int perform_activation_swish_forward(GPUPtr inputPtr, long size, GPUPtr outputPtr, DevicePtr mtlDevicePtr,
                                     CError *err);
int perform_activation_gelu_forward(GPUPtr inputPtr, long size, GPUPtr outputPtr, DevicePtr mtlDevicePtr,
                                    CError *err);

/* MPSGraph calls, metal_bridge.h:1800-1826 (placeholders in the reference,
 * metal_bridge_phase9b.m:82-97, :298-410; Go side gpu/matrix/mps-graph-integration.go).
 * Here a graph of GEMM and activation nodes compiled into a HIP graph:
 *  createMPSGraph      a new, empty graph (NULL on failure);
 *  createMatMulNode    C = A*B of two tensors of the graph (placeholders come from
 *                      gn_graph_placeholder, nodes from these calls); NULL when the inner
 *                      dimensions differ or the data types of A and B differ;
 *  createReLUNode      max(0, x) of an fp32 tensor;
 *  compileGraph        the whole graph: every placeholder is an input (creation order),
 *                      every tensor no node reads is an output (creation order); device is
 *                      ignored (one GPU per process). NULL on failure;
 *  executeCompiledGraph  inputs / outputs are GPUPtr buffers in those orders; runs on the
 *                      stream commandBuffer (NULL: the library stream) and returns after it.
 *                      It reports no error (void, as in the reference): gn_graph_execute does. */
void *createMPSGraph(void);
void *createMatMulNode(void *graph, void *inputA, void *inputB);
void *createReLUNode(void *graph, void *input);
void *compileGraph(void *graph, void *device);
void executeCompiledGraph(void *compiledGraph, void *commandBuffer, void **inputs, long numInputs, void **outputs,
                          long numOutputs);

/* metal_bridge.h:250. */
void free_c_error_message(char *message);

/* ========================================================================== */
/* Part 2 — device-pointer API (no reference counterpart)                      */
/* ========================================================================== */

typedef enum { GN_F32 = 0, GN_F16 = 1 } gn_dtype;
typedef enum { GN_ROUND_NEAREST_EVEN = 0, GN_ROUND_TOWARD_ZERO = 1 } gn_round;
/* Epilogue activations: GN_ACT_NONE plus the Go ActivationType codes. */
enum { GN_ACT_NONE = -1, GN_ACT_RELU = 0, GN_ACT_SIGMOID = 1, GN_ACT_TANH = 2, GN_ACT_LEAKY_RELU = 4,
       GN_ACT_ELU = 5, GN_ACT_SWISH = 6, GN_ACT_GELU = 7 };

/* Drops the index arrays the Part-1 sparse entries keep with values buffer valuesPtr
 * (see perform_sparse_dense_matmul): the next call uploads and validates them again.
 * For callers that change a sparse tensor's index arrays in place. Always 0. */
int gn_csr_indices_changed(GPUPtr valuesPtr);

/* Library version string (static storage). */
const char *gn_version(void);
/* Initialises the device context once (thread-safe). 0 on success. */
int gn_init(CError *err);
/* The library's stream (a hipStream_t, returned as void*). */
void *gn_stream(void);
/* Device pointer of a GPUPtr handle (NULL for an invalid handle), and its size. */
void *gn_buffer_device_ptr(GPUPtr buf);
long gn_buffer_bytes(GPUPtr buf);
/* Live/peak bytes and live allocations of the library's device pool
 * (the GlobalMemoryPool statistics of tensor/tensor.go:65-77). */
void gn_memory_stats(long *current_bytes, long *peak_bytes, long *num_allocations);
/* Device memory from the library pool (caching allocator).
 * gn_free(ptr) waits for the whole device (every stream) and then returns the block to the
 * pool: safe whatever stream used it. It returns -1 and keeps the block when the device
 * cannot be synchronised (a stream capture in progress); free such blocks after the capture.
 * gn_free_async(ptr, stream) does not wait: the block is handed to a new owner only after the
 * work enqueued on `stream` (NULL = the library stream) before the call has finished. Work on
 * other streams that still uses the block must be complete, or ordered before the block's
 * next user (the rule of every stream-ordered allocator). It returns -1 and keeps the block
 * when `stream` is capturing. release_gpu_buffer orders the release on the library stream,
 * where every Part-1 call runs; a caller that uses a GPUPtr's memory on another stream
 * (through gn_buffer_device_ptr) synchronises that stream before releasing the buffer. */
int gn_malloc(void **ptr, size_t bytes, CError *err);
int gn_free(void *ptr);
int gn_free_async(void *ptr, void *stream);
/* Waits for the work enqueued on `stream` (NULL = the library stream), as every synchronous
 * Part-1 call does before it returns: an event recorded behind that work is polled for up to
 * 5 ms, then waited on. -6 with the runtime's message when the work failed, and when `stream`
 * is capturing (a capture has no completion to wait for; the stream and its capture are left
 * as they were). */
int gn_synchronize(void *stream, CError *err);

/* General GEMM on device pointers:
 *   C[M,N] = act( alpha * op(A) * op(B) + beta * C + bias[n] )
 * op(A) is A[M,K] (lda >= K) or, with transA, A stored [K,M] (lda >= M); likewise B.
 * dtype GN_F32: A, B fp32, fp32 MFMA (v_mfma_f32_16x16x4_f32).
 * dtype GN_F16: A, B fp16, fp32 accumulate (v_mfma_f32_16x16x32_f16).
 * C and bias are fp32; bias may be NULL; beta == 0 never reads C.
 * batch >= 1 with element strides strideA/B/C between consecutive problems.
 * Outside HIP graph capture two paths use a scratch block that the library keeps per stream
 * (grown on demand from its pool): operands whose pointer, leading dimension or row length
 * is not a multiple of 16 bytes, in products of at least 2^24 multiply-adds, are first
 * copied into padded K-contiguous buffers, and batch-1 products with few output tiles and a
 * long K are summed over slices of K (partial products, then a reduce in slice order).
 * Under capture neither is taken, and nothing is allocated.
 * Codes: -1 invalid argument, -3 scratch allocation failed, -6 launch error. */
int gn_gemm(int dtype, int transA, int transB, long M, long N, long K, float alpha, const void *A, long lda,
            long strideA, const void *B, long ldb, long strideB, float beta, float *C, long ldc, long strideC,
            long batch, const float *bias, int act, float act_alpha, void *stream, CError *err);

/* fp32 -> fp16 element-wise cast. GN_ROUND_NEAREST_EVEN is IEEE RNE;
 * GN_ROUND_TOWARD_ZERO reproduces Float32ToFloatMP16 (gpu/matrix/mixed-precision.go:106-151)
 * bit for bit, including its fp32-subnormal flush and NaN/overflow handling. */
int gn_cast_f32_f16(const float *in, uint16_t *out, size_t n, int round_mode, void *stream, CError *err);
int gn_cast_f16_f32(const uint16_t *in, float *out, size_t n, void *stream, CError *err);

/* Backward of an element-wise activation applied to a [rows, cols] fp32 pre-activation:
 *   grad_in = (grad_out * act'(pre)) * scale,   grad_bias[j] = sum_i grad_in[i, j]
 * act'(x) is the derivative with respect to the activation's input x, evaluated at pre
 * (codes and formulas as the gn_gemm epilogue; GN_ACT_NONE gives 1). scale carries the
 * dropout factor 1/(1-p) of FusedLinearActivation.Backward (gpu/matrix/fused-operations.go:
 * 528-537; 1 for none). This is steps 1, 2 and 4 of that function (:486-575): the ReLU mask
 * (:491-500), LeakyReLU/Sigmoid/Tanh/GELU backward (:501-520) and the bias gradient
 * ReduceSum(grad, axis 0) (:566-572); step 3 is two gn_gemm calls (NT for grad_input,
 * TN for grad_weight). grad_bias may be NULL; grad_in may alias grad_out. The column sums
 * are added in a fixed order (deterministic). The partial sums go into a per-stream
 * scratch block that the library grows on demand (a larger call releases the old block
 * and allocates a new one), so this call is not for HIP graph capture: a captured graph
 * would keep a block a later, larger call replaces. gn_activation_backward_noalloc is the
 * capturable form. Codes: -1 invalid argument, -3 scratch allocation, -6 launch error. */
int gn_activation_backward(const float *grad_out, const float *pre, long rows, long cols, int act, float alpha,
                           float scale, float *grad_in, float *grad_bias, void *stream, CError *err);

/* No counterpart in the reference. gn_activation_backward for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc. Same arguments and results, bit for bit (same work split and
 * summation order). The partial column sums (chunks x cols floats) go into an 8 MiB
 * device array of the library (each GPU holds its own copy until the process ends)
 * instead of library-allocated scratch; no call allocates or frees memory. Call
 * gn_init() at set-up: it creates the library context and looks up the array's address
 * (the first call of any entry point does so otherwise). Limit: cols <= 2^21 when grad_bias is
 * non-NULL, else -1 with a message. Every call on one GPU shares that array: calls that
 * overlap on one GPU (concurrent streams, or several host threads) race and must be
 * serialised by the caller. Every partial is written before it is read, so no clearing
 * is needed between calls. Codes: -1 invalid argument or too many columns, -6 launch
 * error. */
int gn_activation_backward_noalloc(const float *grad_out, const float *pre, long rows, long cols, int act,
                                   float alpha, float scale, float *grad_in, float *grad_bias, void *stream,
                                   CError *err);

/* out[cols,rows] = in[rows,cols]^T, fp32, LDS-tiled. */
/* out = act(in) element-wise over n floats (the Part-1 activation forwards on device
 * pointers; act is an ActivationType code other than 3, or GN_ACT_NONE to copy). */
int gn_activation_forward(const float *in, float *out, long n, int act, float alpha, void *stream, CError *err);
/* Row-wise softmax of a row-major [rows, cols] fp32 matrix (Softmax in ActivationForward). */
int gn_softmax_rows(const float *in, float *out, long rows, long cols, void *stream, CError *err);
/* Graph extensions (the MPSGraph calls above). gn_graph_placeholder: a rows x cols
 * input of dtype GN_F32 or GN_F16 (fp16 operands of a MatMul must both be fp16; results
 * are fp32). gn_graph_matmul: op(A)*op(B) with transposes (mps-graph-integration.go:151-170
 * passes them; its cgo stub drops them). gn_graph_activation: an element-wise activation
 * (ActivationType code, not Softmax) of an fp32 tensor. gn_graph_compile: the subgraph
 * that computes `outputs` from `inputs` (every placeholder it needs must be an input);
 * a MatMul read only by one activation becomes one GEMM with that activation in its
 * epilogue. gn_graph_execute: copies the inputs in, replays the HIP graph, copies the
 * outputs out, synchronises; executions of one compiled graph are serialised.
 * gn_graph_release: frees a graph or a compiled graph (compiled graphs outlive their
 * graph). Node calls return NULL on invalid arguments. */
void *gn_graph_placeholder(void *graph, long rows, long cols, int dtype);
void *gn_graph_matmul(void *graph, void *inputA, void *inputB, int transA, int transB);
void *gn_graph_activation(void *graph, void *input, int act, float alpha);
int gn_graph_compile(void *graph, void *const *inputs, long numInputs, void *const *outputs, long numOutputs,
                     void **compiled, CError *err);
int gn_graph_execute(void *compiledGraph, void *stream, GPUPtr const *inputs, long numInputs, GPUPtr const *outputs,
                     long numOutputs, CError *err);
void gn_graph_release(void *graphOrCompiled);

int gn_transpose_f32(const float *in, long rows, long cols, float *out, void *stream, CError *err);
/* y[i] += bias[i % len] for i < n: the bias loop of the reference's ForwardFloat16
 * (gpu/matrix/mixed-precision.go:352-354), which adds a bias of any length cyclically over the
 * flat output (the GEMM epilogue covers len == output width). len == 0 with n > 0: -1. */
int gn_add_bias_cyclic_f32(float *y, long n, const float *bias, long len, void *stream, CError *err);

/* CSR SpMM on device arrays: C[M,N] = S[M,K] * D[K,N] (ld = row pitch in elements).
 * Accumulates each output in CSR order with one fused multiply-add per stored entry.
 * error_flags (2 ints, may be NULL) receive nonzero values if a row pointer pair is
 * invalid ([0]) or a column index is outside [0,K) ([1]); offending rows / entries
 * contribute nothing and never cause an out-of-bounds access. From 65536 stored entries
 * (N >= 32, 16-byte aligned rows) it runs as two launches, each row split at its first
 * column >= K/2; outside HIP graph capture the split positions (M ints) go through the
 * library's per-stream scratch, under capture the rows split at the midpoint of their
 * entries instead (no scratch). Either way the result is the same, bit for bit.
 * Codes: -1 invalid argument, -3 scratch allocation failed, -6 launch error. */
int gn_spmm_csr(long M, long N, long K, long nnz, const int32_t *rowptr, const int32_t *col, const float *val,
                const float *D, long ldd, float *C, long ldc, int *error_flags, void *stream, CError *err);
/* CSR SpMV on device arrays: y[M] = S[M,K] * x[K]; error_flags as gn_spmm_csr. */
int gn_spmv_csr(long M, long K, long nnz, const int32_t *rowptr, const int32_t *col, const float *val,
                const float *x, float *y, int *error_flags, void *stream, CError *err);
/* SpMV plan: a one-time analysis of a CSR structure (device arrays) for repeated y = S x
 * with it. No counterpart in the reference; its perform_sparse_matvec gets the same layout
 * through the index arrays kept with the values buffer. Create copies the row pointers to the
 * host and checks them (non-decreasing within [0, nnz]; -1 otherwise), then builds the
 * grouped layout on the device: rows cut into blocks, each block's entries ordered by the
 * 128-byte line of x they gather (6 bytes per stored entry). Run sums each row in CSR order
 * with one fused multiply-add per entry (bit-identical to the reference loop restated with
 * fmaf); error_flags[1] as gn_spmv_csr. rowptr and col must stay unchanged and allocated
 * while the plan lives; values and x may change between runs. Release frees the layout in
 * the order of `stream` (pass the stream of the last run). Codes: -1 invalid argument,
 * -3 allocation failed, -6 launch error. */
int gn_spmv_plan_create(long M, long K, long nnz, const int32_t *rowptr, const int32_t *col, void **plan,
                        void *stream, CError *err);
int gn_spmv_plan_run(const void *plan, const float *val, const float *x, float *y, int *error_flags, void *stream,
                     CError *err);
void gn_spmv_plan_release(void *plan, void *stream);

/* Synthetic data on device: the counter-based SplitMix64 generator
 * (element i of stream s: mix64(seed ^ mix64(s + 0x632BE59BD9B4E019) + (i+1)*0x9E3779B97F4A7C15)),
 * uniform = (u >> 40) * 2^-24 mapped to [lo,hi); normal = Box-Muller (cos branch) in fp64. */
int gn_fill_uniform_f32(float *out, size_t n, uint64_t seed, uint64_t stream_id, float lo, float hi, void *stream,
                        CError *err);
int gn_fill_normal_f32(float *out, size_t n, uint64_t seed, uint64_t stream_id, float mean, float stddev,
                       void *stream, CError *err);

/* ========================================================================== */
/* Part 3 — the rest of internal/cgo/metal_bridge.h that the Go packages bind  */
/* ========================================================================== */
/* Every function that a non-test file of gpu/matrix, gpu/optimizer or tensor calls through
 * cgo is declared here with the reference prototype, so that those packages compile and
 * link against this library (tests/golden/cgo_abi.json lists each one with its reference
 * header line and Go call sites). The element-wise matrix operations and the activation
 * backwards below are device implementations; the groups after them belong to subsystems
 * this backend does not cover and return -1 with the message "<name>: not provided by the
 * go-nngpu MI355X GEMM/SpMM backend" in *err. */

/* metal_bridge.h:7-16 types that Go code names (C.GPUCounters, C.KernelCompileOptions). */
typedef void *CommandQueuePtr; /* metal_bridge.h:11 */
typedef struct {               /* metal_bridge.h:1701-1708 */
  int optimization_level;
  bool fast_math;
  bool debug_info;
  int num_constants;
  int num_macros;
} KernelCompileOptions;
typedef struct { /* metal_bridge.h:1810-1814 */
  float computeUtilization;
  float memoryBandwidth;
  float cacheHitRate;
} GPUCounters;

/* Element-wise matrix operations (gpu/matrix/matrix.go calls at :486 add, :530 add_broadcast,
 * :581 subtract, :632 element_multiply, :683 element_divide, :727 scalar_add, :771
 * scalar_multiply; reference loops metal_bridge_matrix.m:172-543).
 * fp32, one rounding per operation as written: result = a + b, a - b, a * b, a / b
 * (IEEE, correctly rounded), input + scalar, input * scalar. The result buffer may be one of
 * the inputs. mtlDevicePtr may be NULL. Synchronous.
 *  add / subtract / element_multiply / element_divide: -2 unless aRows == bRows == resultRows
 *    and aCols == bCols == resultCols (:180-183), -3 NULL or too small buffer (:215-218).
 *  element_divide: -4 "Division by zero encountered at element <i>." with the lowest such i
 *    (:470-474); the reference stops at that element, here every element is written.
 *  add_broadcast: [M,N] + [1,N], [1,N] + [M,N], [M,N] + [M,1], [M,1] + [M,N] -> [M,N],
 *    tried in that order (:267-311); another shape combination -2, NULL or too small
 *    buffer -3.
 *  scalar_add / scalar_multiply: -1 NULL or too small buffer (:492-495).
 *  All: -1 on a device execution error. */
int perform_mps_matrix_add(GPUPtr aMatrixPtr, long aRows, long aCols, GPUPtr bMatrixPtr, long bRows, long bCols,
                           GPUPtr resultMatrixPtr, long resultRows, long resultCols, DevicePtr mtlDevicePtr,
                           CError *err);
int perform_mps_matrix_add_broadcast(GPUPtr aMatrixPtr, long aRows, long aCols, GPUPtr bMatrixPtr, long bRows,
                                     long bCols, GPUPtr resultMatrixPtr, long resultRows, long resultCols,
                                     DevicePtr mtlDevicePtr, CError *err);
int perform_mps_matrix_element_divide(GPUPtr aMatrixPtr, long aRows, long aCols, GPUPtr bMatrixPtr, long bRows,
                                      long bCols, GPUPtr resultMatrixPtr, long resultRows, long resultCols,
                                      DevicePtr mtlDevicePtr, CError *err);
int perform_mps_matrix_element_multiply(GPUPtr aMatrixPtr, long aRows, long aCols, GPUPtr bMatrixPtr, long bRows,
                                        long bCols, GPUPtr resultMatrixPtr, long resultRows, long resultCols,
                                        DevicePtr mtlDevicePtr, CError *err);
int perform_mps_matrix_scalar_add(GPUPtr inputMatrixPtr, long rows, long cols, float scalar, GPUPtr resultMatrixPtr,
                                  DevicePtr mtlDevicePtr, CError *err);
int perform_mps_matrix_scalar_multiply(GPUPtr inputMatrixPtr, long rows, long cols, float scalar,
                                       GPUPtr resultMatrixPtr, DevicePtr mtlDevicePtr, CError *err);
int perform_mps_matrix_subtract(GPUPtr aMatrixPtr, long aRows, long aCols, GPUPtr bMatrixPtr, long bRows,
                                long bCols, GPUPtr resultMatrixPtr, long resultRows, long resultCols,
                                DevicePtr mtlDevicePtr, CError *err);
/* Activation backward (gpu/matrix/activation.go ActivationBackward :177-300, calls at
 * :223-283, called by
 * FusedLinearActivation.Backward, fused-operations.go:486-523). Each takes the gradient with
 * respect to the activation's output and the activation OUTPUT y (not its input), over
 * `size` floats, and computes the reference's formulas (metal_bridge_activation.m) in fp32
 * with one rounding per operation as written:
 *   ReLU       gradIn = y > 0 ? g : 0                                   (:54-82)
 *   Sigmoid    gradIn = g * y * (1 - y)                                 (:114-143)
 *   Tanh       gradIn = g * (1 - y * y)                                 (:175-204)
 *   LeakyReLU  gradIn = g * (y > 0 ? 1 : alpha)                         (:401-433)
 *   ELU        gradIn = g * (y > 0 ? 1 : y + alpha)                     (:471-512)
 *   Swish      x from y by three Newton steps on x*sigmoid(x) = y from x = y (a step is
 *              skipped where |f'| <= 1e-8); gradIn = g * (s + x s (1 - s)), s = sigmoid(x);
 *              |y| < 1e-8 gives g * 0.5                                 (:546-604)
 *   GELU       x from y by three Newton steps on GELU(x) = y from x = y (tanh form, inner
 *              argument clamped to [-88, 88]); gradIn = g * GELU'(x)    (:642-702)
 *   Softmax    gradIn = y * (g - dot(g, y)), over all `size` values (1-D, :247-281) or per
 *              row of [batchSize, features] (2-D, :329-369); the dot products are summed in
 *              a fixed tree order, not the reference's sequential one.
 * Sigmoid, Swish and GELU use expf / tanhf (within a few ulp of the C library's). gradIn
 * may alias either input. Codes: -1 NULL or too small buffer, negative size, or execution
 * error (the reference's -1 for bad buffers). */
int perform_activation_elu_backward(GPUPtr gradOutputPtr, GPUPtr activationOutputPtr, long size, float alpha,
                                    GPUPtr gradInputPtr, DevicePtr mtlDevicePtr, CError *err);
int perform_activation_gelu_backward(GPUPtr gradOutputPtr, GPUPtr activationOutputPtr, long size,
                                     GPUPtr gradInputPtr, DevicePtr mtlDevicePtr, CError *err);
int perform_activation_leaky_relu_backward(GPUPtr gradOutputPtr, GPUPtr activationOutputPtr, long size, float alpha,
                                           GPUPtr gradInputPtr, DevicePtr mtlDevicePtr, CError *err);
int perform_activation_relu_backward(GPUPtr gradOutputPtr, GPUPtr activationOutputPtr, long size,
                                     GPUPtr gradInputPtr, DevicePtr mtlDevicePtr, CError *err);
int perform_activation_sigmoid_backward(GPUPtr gradOutputPtr, GPUPtr activationOutputPtr, long size,
                                        GPUPtr gradInputPtr, DevicePtr mtlDevicePtr, CError *err);
int perform_activation_softmax_1d_backward(GPUPtr gradOutputPtr, GPUPtr activationOutputPtr, long size,
                                           GPUPtr gradInputPtr, DevicePtr mtlDevicePtr, CError *err);
int perform_activation_softmax_2d_backward(GPUPtr gradOutputPtr, GPUPtr activationOutputPtr, long batchSize,
                                           long features, GPUPtr gradInputPtr, DevicePtr mtlDevicePtr, CError *err);
int perform_activation_swish_backward(GPUPtr gradOutputPtr, GPUPtr activationOutputPtr, long size,
                                      GPUPtr gradInputPtr, DevicePtr mtlDevicePtr, CError *err);
int perform_activation_tanh_backward(GPUPtr gradOutputPtr, GPUPtr activationOutputPtr, long size,
                                     GPUPtr gradInputPtr, DevicePtr mtlDevicePtr, CError *err);
/* Dense decompositions (matrix.go: Inverse, Determinant, LU, QR, Cholesky, Eigen, SVD; the
 * reference runs LAPACK on the CPU, metal_bridge_decomposition.m). Not provided: -1. */
/* metal_bridge.h:137; gpu/matrix/matrix.go:137 */
int perform_matrix_cholesky_decomposition(GPUPtr inputMatrixPtr, long rows, long cols, GPUPtr lMatrixPtr,
                                          DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:110; gpu/matrix/matrix.go:859 */
int perform_matrix_determinant(GPUPtr inputMatrixPtr, long rows, long cols, float *determinant,
                               DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:145; gpu/matrix/matrix.go:218 */
int perform_matrix_eigenvalue_decomposition(GPUPtr inputMatrixPtr, long rows, long cols, GPUPtr eigenvaluesPtr,
                                            GPUPtr eigenvectorsPtr, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:102; gpu/matrix/matrix.go:822 */
int perform_matrix_inverse(GPUPtr inputMatrixPtr, long rows, long cols, GPUPtr resultMatrixPtr,
                           DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:118; gpu/matrix/matrix.go:949 */
int perform_matrix_lu_decomposition(GPUPtr inputMatrixPtr, long rows, long cols, GPUPtr lMatrixPtr,
                                    GPUPtr uMatrixPtr, int *pivotIndices, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:129; gpu/matrix/matrix.go:1037 */
int perform_matrix_qr_decomposition(GPUPtr inputMatrixPtr, long rows, long cols, GPUPtr qMatrixPtr,
                                    GPUPtr rMatrixPtr, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:154; gpu/matrix/matrix.go:328 */
int perform_matrix_svd_decomposition(GPUPtr inputMatrixPtr, long rows, long cols, GPUPtr uMatrixPtr,
                                     GPUPtr sVectorPtr, GPUPtr vtMatrixPtr, DevicePtr mtlDevicePtr, CError *err);

/* Loss functions (loss.go; CPU loops in metal_bridge_loss.m). Not provided: -1. */
/* metal_bridge.h:422; gpu/matrix/loss.go:259 */
int perform_loss_binary_crossentropy_backward(GPUPtr predictionsPtr, GPUPtr targetsPtr, long size,
                                              GPUPtr gradInputPtr, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:415; gpu/matrix/loss.go:117 */
int perform_loss_binary_crossentropy_forward(GPUPtr predictionsPtr, GPUPtr targetsPtr, long size, float *loss,
                                             DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:437; gpu/matrix/loss.go:272 */
int perform_loss_categorical_crossentropy_backward(GPUPtr predictionsPtr, GPUPtr targetsPtr, long batchSize,
                                                   long numClasses, GPUPtr gradInputPtr, DevicePtr mtlDevicePtr,
                                                   CError *err);
/* metal_bridge.h:430; gpu/matrix/loss.go:130 */
int perform_loss_categorical_crossentropy_forward(GPUPtr predictionsPtr, GPUPtr targetsPtr, long batchSize,
                                                  long numClasses, float *loss, DevicePtr mtlDevicePtr,
                                                  CError *err);
/* metal_bridge.h:499; gpu/matrix/loss.go:314 */
int perform_loss_hinge_backward(GPUPtr predictionsPtr, GPUPtr targetsPtr, long size, GPUPtr gradInputPtr,
                                DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:492; gpu/matrix/loss.go:172 */
int perform_loss_hinge_forward(GPUPtr predictionsPtr, GPUPtr targetsPtr, long size, float *loss,
                               DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:468; gpu/matrix/loss.go:289 */
int perform_loss_huber_backward(GPUPtr predictionsPtr, GPUPtr targetsPtr, long size, float delta,
                                GPUPtr gradInputPtr, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:460; gpu/matrix/loss.go:147 */
int perform_loss_huber_forward(GPUPtr predictionsPtr, GPUPtr targetsPtr, long size, float delta, float *loss,
                               DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:484; gpu/matrix/loss.go:302 */
int perform_loss_mae_backward(GPUPtr predictionsPtr, GPUPtr targetsPtr, long size, GPUPtr gradInputPtr,
                              DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:477; gpu/matrix/loss.go:160 */
int perform_loss_mae_forward(GPUPtr predictionsPtr, GPUPtr targetsPtr, long size, float *loss,
                             DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:407; gpu/matrix/loss.go:247 */
int perform_loss_mse_backward(GPUPtr predictionsPtr, GPUPtr targetsPtr, long size, GPUPtr gradInputPtr,
                              DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:400; gpu/matrix/loss.go:105 */
int perform_loss_mse_forward(GPUPtr predictionsPtr, GPUPtr targetsPtr, long size, float *loss,
                             DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:452; gpu/matrix/loss.go:451 */
int perform_loss_sparse_categorical_crossentropy_backward(GPUPtr predictionsPtr, int *targetIndices, long batchSize,
                                                          long numClasses, GPUPtr gradInputPtr,
                                                          DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:445; gpu/matrix/loss.go:388 */
int perform_loss_sparse_categorical_crossentropy_forward(GPUPtr predictionsPtr, int *targetIndices, long batchSize,
                                                         long numClasses, float *loss, DevicePtr mtlDevicePtr,
                                                         CError *err);

/* Apple memory-pool and buffer-placement helpers (memory-pool.go, memory-optimization.go;
 * metal_bridge_memory.m). Buffers come from create_gpu_buffer and the gn_malloc pool here.
 * Not provided: -1. */
/* metal_bridge.h:1495; gpu/matrix/memory-optimization.go:30 */
int allocate_aligned_gpu_buffer(long size, long alignment, GPUPtr *bufferPtr, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:1383; gpu/matrix/memory-pool.go:157 */
int allocate_gpu_memory(long size, GPUPtr *ptr, CError *error);
/* metal_bridge.h:1385; gpu/matrix/memory-pool.go:354 */
int cleanup_memory_pool(CError *error);
/* metal_bridge.h:1510; gpu/matrix/memory-optimization.go:67 */
int coalesced_memory_copy(GPUPtr srcPtr, GPUPtr dstPtr, long size, long srcStride, long dstStride,
                          DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:1530; gpu/matrix/memory-optimization.go:104 */
int flush_gpu_cache(DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:1384; gpu/matrix/memory-pool.go:244 (+1 more) */
int free_gpu_memory(GPUPtr ptr, CError *error);
/* metal_bridge.h:1382; gpu/matrix/memory-pool.go:100 */
int initialize_memory_pool(long max_memory, CError *error);
/* metal_bridge.h:1521; gpu/matrix/memory-optimization.go:86 */
int prefetch_gpu_data(GPUPtr bufferPtr, long size, long offset, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:1504; gpu/matrix/memory-optimization.go:49 */
int release_optimized_gpu_buffer(GPUPtr bufferPtr, CError *err);

/* Convolution, pooling, padding, im2col (convolution.go; metal_bridge_convolution.m).
 * Not provided: -1. */
/* metal_bridge.h:571; gpu/matrix/convolution.go:533 */
int perform_avgpool2d_backward(GPUPtr gradOutputPtr, long gradOutputBatch, long gradOutputHeight,
                               long gradOutputWidth, long gradOutputChannels, GPUPtr gradInputPtr,
                               long gradInputBatch, long gradInputHeight, long gradInputWidth,
                               long gradInputChannels, long poolHeight, long poolWidth, long strideH, long strideW,
                               long padH, long padW, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:562; gpu/matrix/convolution.go:477 */
int perform_avgpool2d_forward(GPUPtr inputPtr, long inputBatch, long inputHeight, long inputWidth,
                              long inputChannels, GPUPtr outputPtr, long outputBatch, long outputHeight,
                              long outputWidth, long outputChannels, long poolHeight, long poolWidth, long strideH,
                              long strideW, long padH, long padW, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:609; gpu/matrix/convolution.go:783 */
int perform_col2im(GPUPtr inputPtr, GPUPtr outputPtr, long outputBatch, long outputHeight, long outputWidth,
                   long outputChannels, long kernelHeight, long kernelWidth, long strideH, long strideW, long padH,
                   long padW, long inputHeight, long inputWidth, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:522; gpu/matrix/convolution.go:210 */
int perform_conv2d_backward_input(GPUPtr gradOutputPtr, long gradOutputBatch, long gradOutputHeight,
                                  long gradOutputWidth, long gradOutputChannels, GPUPtr kernelPtr,
                                  long kernelHeight, long kernelWidth, long kernelInputChannels,
                                  long kernelOutputChannels, GPUPtr gradInputPtr, long gradInputBatch,
                                  long gradInputHeight, long gradInputWidth, long gradInputChannels, long strideH,
                                  long strideW, long padH, long padW, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:532; gpu/matrix/convolution.go:283 */
int perform_conv2d_backward_kernel(GPUPtr inputPtr, long inputBatch, long inputHeight, long inputWidth,
                                   long inputChannels, GPUPtr gradOutputPtr, long gradOutputBatch,
                                   long gradOutputHeight, long gradOutputWidth, long gradOutputChannels,
                                   GPUPtr gradKernelPtr, long kernelHeight, long kernelWidth,
                                   long kernelInputChannels, long kernelOutputChannels, long strideH, long strideW,
                                   long padH, long padW, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:512; gpu/matrix/convolution.go:137 */
int perform_conv2d_forward(GPUPtr inputPtr, long inputBatch, long inputHeight, long inputWidth, long inputChannels,
                           GPUPtr kernelPtr, long kernelHeight, long kernelWidth, long kernelInputChannels,
                           long kernelOutputChannels, GPUPtr outputPtr, long outputBatch, long outputHeight,
                           long outputWidth, long outputChannels, long strideH, long strideW, long padH, long padW,
                           DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:599; gpu/matrix/convolution.go:722 */
int perform_im2col(GPUPtr inputPtr, long inputBatch, long inputHeight, long inputWidth, long inputChannels,
                   GPUPtr outputPtr, long kernelHeight, long kernelWidth, long strideH, long strideW, long padH,
                   long padW, long outputHeight, long outputWidth, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:552; gpu/matrix/convolution.go:415 */
int perform_maxpool2d_backward(GPUPtr gradOutputPtr, long gradOutputBatch, long gradOutputHeight,
                               long gradOutputWidth, long gradOutputChannels, GPUPtr indicesPtr,
                               GPUPtr gradInputPtr, long gradInputBatch, long gradInputHeight, long gradInputWidth,
                               long gradInputChannels, long poolHeight, long poolWidth, long strideH, long strideW,
                               long padH, long padW, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:542; gpu/matrix/convolution.go:355 */
int perform_maxpool2d_forward(GPUPtr inputPtr, long inputBatch, long inputHeight, long inputWidth,
                              long inputChannels, GPUPtr outputPtr, long outputBatch, long outputHeight,
                              long outputWidth, long outputChannels, GPUPtr indicesPtr, long poolHeight,
                              long poolWidth, long strideH, long strideW, long padH, long padW,
                              DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:580; gpu/matrix/convolution.go:595 */
int perform_pad2d(GPUPtr inputPtr, long inputBatch, long inputHeight, long inputWidth, long inputChannels,
                  GPUPtr outputPtr, long outputBatch, long outputHeight, long outputWidth, long outputChannels,
                  long padTop, long padBottom, long padLeft, long padRight, float padValue, DevicePtr mtlDevicePtr,
                  CError *err);
/* metal_bridge.h:590; gpu/matrix/convolution.go:658 */
int perform_unpad2d(GPUPtr inputPtr, long inputBatch, long inputHeight, long inputWidth, long inputChannels,
                    GPUPtr outputPtr, long outputBatch, long outputHeight, long outputWidth, long outputChannels,
                    long padTop, long padBottom, long padLeft, long padRight, DevicePtr mtlDevicePtr, CError *err);

/* Batch / layer / group / instance normalisation (batch-norm.go; metal_bridge_normalization.m).
 * Not provided: -1. */
/* metal_bridge.h:621; gpu/matrix/batch-norm.go:111 */
int perform_batch_mean(GPUPtr inputPtr, long batchSize, long features, GPUPtr meanPtr, DevicePtr mtlDevicePtr,
                       CError *err);
/* metal_bridge.h:648; gpu/matrix/batch-norm.go:304 */
int perform_batch_norm_backward_input(GPUPtr gradOutputPtr, long batchSize, long features, GPUPtr inputPtr,
                                      GPUPtr meanPtr, GPUPtr variancePtr, GPUPtr gammaPtr, float epsilon,
                                      GPUPtr gradInputPtr, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:658; gpu/matrix/batch-norm.go:323 */
int perform_batch_norm_backward_params(GPUPtr gradOutputPtr, long batchSize, long features, GPUPtr inputPtr,
                                       GPUPtr meanPtr, GPUPtr variancePtr, float epsilon, GPUPtr gradGammaPtr,
                                       GPUPtr gradBetaPtr, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:637; gpu/matrix/batch-norm.go:239 */
int perform_batch_norm_forward(GPUPtr inputPtr, long batchSize, long features, GPUPtr meanPtr, GPUPtr variancePtr,
                               GPUPtr gammaPtr, GPUPtr betaPtr, float epsilon, GPUPtr outputPtr,
                               DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:629; gpu/matrix/batch-norm.go:165 */
int perform_batch_variance(GPUPtr inputPtr, GPUPtr meanPtr, long batchSize, long features, GPUPtr variancePtr,
                           DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:716; gpu/matrix/batch-norm.go:608 */
int perform_group_norm_forward(GPUPtr inputPtr, long batchSize, long channels, long height, long width,
                               long numGroups, GPUPtr gammaPtr, GPUPtr betaPtr, float epsilon, GPUPtr outputPtr,
                               DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:697; gpu/matrix/batch-norm.go:553 */
int perform_instance_norm_forward(GPUPtr inputPtr, long batchSize, long channels, long height, long width,
                                  GPUPtr gammaPtr, GPUPtr betaPtr, float epsilon, GPUPtr outputPtr,
                                  DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:678; gpu/matrix/batch-norm.go:455 */
int perform_layer_norm_backward(GPUPtr gradOutputPtr, long batchSize, long features, GPUPtr inputPtr,
                                GPUPtr meanPtr, GPUPtr variancePtr, GPUPtr gammaPtr, float epsilon,
                                GPUPtr gradInputPtr, GPUPtr gradGammaPtr, GPUPtr gradBetaPtr,
                                DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:668; gpu/matrix/batch-norm.go:389 */
int perform_layer_norm_forward(GPUPtr inputPtr, long batchSize, long features, GPUPtr gammaPtr, GPUPtr betaPtr,
                               float epsilon, GPUPtr outputPtr, GPUPtr meanPtr, GPUPtr variancePtr,
                               DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:688; gpu/matrix/batch-norm.go:503 */
int perform_update_running_stats(GPUPtr runningMeanPtr, GPUPtr runningVarPtr, GPUPtr batchMeanPtr,
                                 GPUPtr batchVarPtr, float momentum, long features, DevicePtr mtlDevicePtr,
                                 CError *err);

/* Fused operations other than the linear layer (fused-operations.go; metal_bridge_fused.m).
 * Not provided: -1. */
/* metal_bridge.h:1355; gpu/matrix/fused-operations.go:645 */
int perform_fused_attention(GPUPtr query, GPUPtr key, GPUPtr value, long batch_size, long seq_len, long model_dim,
                            int num_heads, float scale, float dropout_rate, bool causal, GPUPtr output,
                            DevicePtr device, CError *error);
/* metal_bridge.h:1338; gpu/matrix/fused-operations.go:241 */
int perform_fused_conv_bn_relu(GPUPtr input, long batch_size, long input_h, long input_w, long input_channels,
                               GPUPtr kernel, long kernel_h, long kernel_w, long output_channels, GPUPtr gamma,
                               GPUPtr beta, GPUPtr bias, long stride_h, long stride_w, long pad_h, long pad_w,
                               float epsilon, bool training, GPUPtr output, long output_h, long output_w,
                               DevicePtr device, CError *error);
/* metal_bridge.h:1362; gpu/matrix/fused-operations.go:873 */
int perform_fused_gelu_dropout(GPUPtr input, long size, float dropout_rate, unsigned int seed, GPUPtr output,
                               DevicePtr device, CError *error);
/* metal_bridge.h:1367; gpu/matrix/fused-operations.go:1047 */
int perform_fused_layer_norm_linear(GPUPtr input, long batch_size, long seq_len, long input_dim, GPUPtr gamma,
                                    GPUPtr beta, float epsilon, GPUPtr weight, long output_dim, GPUPtr bias,
                                    GPUPtr output, DevicePtr device, CError *error);
/* metal_bridge.h:1374; gpu/matrix/fused-operations.go:1234 */
int perform_fused_residual_block(GPUPtr input, long batch_size, long height, long width, long channels,
                                 GPUPtr conv1_weight, GPUPtr bn1_gamma, GPUPtr bn1_beta, GPUPtr conv2_weight,
                                 GPUPtr bn2_gamma, GPUPtr bn2_beta, float epsilon, GPUPtr output, DevicePtr device,
                                 CError *error);

/* Embedded-MSL kernels other than the GEMMs (optimized-kernels.go; metal_bridge_kernels.m).
 * Not provided: -1. */
/* metal_bridge.h:1440; gpu/matrix/optimized-kernels.go:178 */
int perform_conv1x1_optimized(GPUPtr inputPtr, GPUPtr weightPtr, GPUPtr outputPtr, long batch, long height,
                              long width, long inChannels, long outChannels, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:1449; gpu/matrix/optimized-kernels.go:244 */
int perform_depthwise_conv_optimized(GPUPtr inputPtr, GPUPtr kernelPtr, GPUPtr outputPtr, long batch, long inHeight,
                                     long inWidth, long channels, long kernelH, long kernelW, long strideH,
                                     long strideW, long padH, long padW, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:1459; gpu/matrix/optimized-kernels.go:310 */
int perform_elementwise_binary_op_optimized(GPUPtr aPtr, GPUPtr bPtr, GPUPtr outputPtr, int opType, long size,
                                            long aStride, long bStride, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:1484; gpu/matrix/optimized-kernels.go:466 */
int perform_layer_norm_optimized(GPUPtr inputPtr, GPUPtr gammaPtr, GPUPtr betaPtr, GPUPtr outputPtr,
                                 GPUPtr meanOutPtr, GPUPtr varOutPtr, long batchSize, long featureSize,
                                 float epsilon, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:1468; gpu/matrix/optimized-kernels.go:352 */
int perform_reduce_optimized(GPUPtr inputPtr, GPUPtr outputPtr, long size, int opType, DevicePtr mtlDevicePtr,
                             CError *err);
/* metal_bridge.h:1476; gpu/matrix/optimized-kernels.go:399 */
int perform_softmax_optimized(GPUPtr inputPtr, GPUPtr outputPtr, long batchSize, long numClasses,
                              DevicePtr mtlDevicePtr, CError *err);

/* Gradient utilities (gradient.go, grad-ops.go, training.go; metal_bridge_gradient.m).
 * Not provided: -1. */
/* metal_bridge.h:1415; gpu/matrix/grad-ops.go:234 */
int perform_dropout_backward(GPUPtr grad_output, GPUPtr mask, long size, float probability, GPUPtr grad_input,
                             DevicePtr device, CError *error);
/* metal_bridge.h:1410; gpu/matrix/grad-ops.go:190 */
int perform_dropout_forward(GPUPtr input, long size, float probability, unsigned int seed, GPUPtr output,
                            GPUPtr mask, DevicePtr device, CError *error);
/* metal_bridge.h:1388; gpu/matrix/gradient.go:283 */
int perform_gradient_accumulate(GPUPtr existing_grad, GPUPtr new_grad, long size, DevicePtr device, CError *error);
/* metal_bridge.h:1398; gpu/matrix/gradient.go:914 */
int perform_sum_along_axis(GPUPtr input, int axis, long input_ndim, long *input_shape, GPUPtr output,
                           long output_ndim, long *output_shape, DevicePtr device, CError *error);
/* metal_bridge.h:1404; gpu/matrix/training.go:894 (+4 more) */
int perform_tensor_fill(GPUPtr tensor, long size, float value, DevicePtr device, CError *error);
/* metal_bridge.h:1393; gpu/matrix/gradient.go:374 */
int perform_tensor_sum_squares(GPUPtr tensor, long size, float *result, DevicePtr device, CError *error);

/* Optimizer steps, clipping and learning-rate schedules (package gpu/optimizer;
 * metal_bridge_optimizer.m). Not provided: -1. */
/* metal_bridge.h:990; gpu/optimizer/optimizer.go:256 */
int perform_adam_step(GPUPtr paramsPtr, GPUPtr gradPtr, long size, float learningRate, float beta1, float beta2,
                      float epsilon, float weightDecay, GPUPtr m_bufferPtr, GPUPtr v_bufferPtr, long stepNumber,
                      DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:1050; gpu/optimizer/optimizer.go:606 */
int perform_adamw_step(GPUPtr paramsPtr, GPUPtr gradPtr, long size, float learningRate, float beta1, float beta2,
                       float epsilon, float weightDecay, GPUPtr m_bufferPtr, GPUPtr v_bufferPtr, long stepNumber,
                       DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:1142; gpu/optimizer/optimizer.go:730 */
int perform_global_gradient_clip(GPUPtr *gradPtrs, long *sizes, long numTensors, float maxNorm, float *actualNorm,
                                 DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:1132; gpu/optimizer/optimizer.go:810 */
int perform_global_gradient_norm(GPUPtr *gradPtrs, long *sizes, long numTensors, float *globalNorm,
                                 DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:1122; gpu/optimizer/optimizer.go:761 */
int perform_gradient_clip_by_value(GPUPtr gradPtr, long size, float minValue, float maxValue,
                                   DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:1089; gpu/optimizer/scheduler.go:167 */
int perform_lr_cosine_annealing(float *currentLR, float initialLR, float minLR, long stepNumber, long totalSteps,
                                CError *err);
/* metal_bridge.h:1069; gpu/optimizer/scheduler.go:47 */
int perform_lr_exponential_decay(float *currentLR, float initialLR, float decayRate, long stepNumber,
                                 long decaySteps, CError *err);
/* metal_bridge.h:1099; gpu/optimizer/scheduler.go:229 */
int perform_lr_polynomial_decay(float *currentLR, float initialLR, float finalLR, long stepNumber, long totalSteps,
                                float power, CError *err);
/* metal_bridge.h:1079; gpu/optimizer/scheduler.go:107 */
int perform_lr_step_decay(float *currentLR, float initialLR, float gamma, long stepNumber, long stepSize,
                          CError *err);
/* metal_bridge.h:1201; gpu/optimizer/scheduler.go:296 */
int perform_lr_warmup(float *currentLR, float targetLR, long stepNumber, long warmupSteps, int warmupType,
                      CError *err);
/* metal_bridge.h:1007; gpu/optimizer/optimizer.go:436 */
int perform_rmsprop_step(GPUPtr paramsPtr, GPUPtr gradPtr, long size, float learningRate, float alpha,
                         float epsilon, float momentum, float weightDecay, GPUPtr squaredGradBufferPtr,
                         GPUPtr momentumBufferPtr, DevicePtr mtlDevicePtr, CError *err);
/* metal_bridge.h:977; gpu/optimizer/optimizer.go:97 */
int perform_sgd_step(GPUPtr paramsPtr, GPUPtr gradPtr, long size, float learningRate, float momentum,
                     GPUPtr momentumBufferPtr, float weightDecay, DevicePtr mtlDevicePtr, CError *err);

/* Command queues, events, shared / mapped memory, counters and the MPSGraph convolution
 * node (multi-stream-execution.go, unified-memory-optimization.go, command-queue-pool.go,
 * profiling-autotuning.go, mps-graph-integration.go; metal_bridge_phase9b.m, whose own
 * versions are placeholders). Pointer results are NULL (memoryMapFile also sets *error),
 * void calls do nothing, getGPUCounters stores zeros, getGPUPowerUsage and
 * getGPUTemperature return 0. getGPUMemoryUsage reports the device's total and used HBM
 * (hipMemGetInfo). */
/* metal_bridge.h:1803; gpu/matrix/unified-memory-optimization.go:476 */
void *allocateSharedMemory(long size);
/* metal_bridge.h:1797; gpu/matrix/command-queue-pool.go:53 (+2 more) */
void *createCommandQueue(void *device);
/* metal_bridge.h:1823; gpu/matrix/mps-graph-integration.go:582 */
void *createConv2DNode(void *graph, void *input, void *weights, long strideH, long strideW, long padH, long padW);
/* metal_bridge.h:1804; gpu/matrix/unified-memory-optimization.go:486 */
void *createGPUBufferFromSharedMemory(void *device, void *sharedMemory, long size);
/* metal_bridge.h:1799; gpu/matrix/multi-stream-execution.go:351 */
void *createMetalEvent(void *device);
/* metal_bridge.h:1816; gpu/matrix/profiling-autotuning.go:782 (+1 more) */
void getGPUCounters(GPUCounters *counters);
/* metal_bridge.h:1817; gpu/matrix/profiling-autotuning.go:769 (+1 more) */
void getGPUMemoryUsage(long *totalBytes, long *usedBytes);
/* metal_bridge.h:1818; gpu/matrix/profiling-autotuning.go:794 */
float getGPUPowerUsage(void);
/* metal_bridge.h:1819; gpu/matrix/profiling-autotuning.go:803 */
float getGPUTemperature(void);
/* metal_bridge.h:1805; gpu/matrix/unified-memory-optimization.go:530 */
void makeBufferGPUResident(void *buffer);
/* metal_bridge.h:1806; gpu/matrix/unified-memory-optimization.go:496 */
void *memoryMapFile(const char *path, long *size, CError *error);
/* metal_bridge.h:1798; gpu/matrix/multi-stream-execution.go:347 */
void synchronizeCommandQueue(void *queue);
/* metal_bridge.h:1807; gpu/matrix/unified-memory-optimization.go:512 */
void unmapMemory(void *memory, long size);

#ifdef __cplusplus
}
#endif
#endif /* GONNGPU_H */
