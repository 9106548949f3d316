/*
 * oracle.h — CPU restatement of the reference's GEMM / fp16 / CSR / SpMM / SpMV
 * semantics, used ONLY as the checker by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py. Nothing in the product path links or calls it.
 *
 * Every function names the reference file:line it restates (paths relative to the
 * reference repository root, module github.com/tsawler/gometal).
 *
 * Pins (what checks each function against something other than itself) are listed
 * per function; the tests live in tests/test_oracle.py.
 */
#ifndef GONNGPU_ORACLE_H
#define GONNGPU_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- deterministic synthetic data --------------------------------------- */
/* Counter-based SplitMix64: element i of stream s under seed is
 * mix64(seed ^ mix64(s) + (i+1)*0x9E3779B97F4A7C15). Uniform = (u>>40)*2^-24 in
 * [0,1). Normal = Box–Muller (cos branch) in float64 from the uniforms of counters
 * 2i and 2i+1, rounded to fp32. Identical formulas run on the GPU bench path. */
uint64_t orc_splitmix64(uint64_t seed, uint64_t stream, uint64_t i);
void orc_fill_uniform_f32(float *out, size_t n, uint64_t seed, uint64_t stream, float lo, float hi);
void orc_fill_normal_f32(float *out, size_t n, uint64_t seed, uint64_t stream, float mean, float stddev);

/* ---- dense GEMM (gonum mat.Dense.Mul semantics, float64) --------------- */
/* C[M,N] = alpha * op(A)[M,K] * op(B)[K,N] + beta * C, inputs fp32 (exactly widened),
 * accumulation and output in float64. op(X) = X (trans=0) or X^T (trans=1); all
 * matrices row-major with leading dimension ld*. Restates BLAS dgemm / gonum
 * mat.Dense.Mul (gonum v0.16.0, not vendored) as used at
 * gpu/matrix/gonum-compat.go:342-367 and internal/cgo/metal_bridge_matrix.m:90-97
 * (alpha=1, beta=0), and the alpha/beta form of metal_bridge_kernels.m:81.
 * Pins: numpy float64 matmul, closed forms, transpose identities. */
void orc_gemm_f64(int transA, int transB, long M, long N, long K, double alpha,
                  const float *A, long lda, const float *B, long ldb, double beta,
                  double *C, long ldc, int threads);
/* Same, but only for the listed output rows (rows[r] in [0,M)); C has nrows rows. */
void orc_gemm_f64_rows(int transA, int transB, long M, long N, long K,
                       const float *A, long lda, const float *B, long ldb,
                       const long *rows, long nrows, double *C, long ldc, int threads);

/* ---- fp16 conversion ----------------------------------------------------- */
/* Bit-exact restatement of Float32ToFloatMP16, gpu/matrix/mixed-precision.go:106-151:
 * truncation toward zero, fp32 subnormals -> signed zero, overflow -> inf,
 * NaN -> 0x7C00|(mant>>13) (so a NaN whose top 10 payload bits are 0 becomes inf).
 * Pins: IEEE round-toward-zero computed from numpy float16 + nextafter, special table. */
uint16_t orc_f32_to_f16_rtz(float f);
/* Bit-exact restatement of FloatMP16ToFloat32, mixed-precision.go:154-189 (exact widening).
 * Pins: numpy float16 -> float32 over all 65536 patterns. */
float orc_f16_to_f32(uint16_t h);
/* IEEE 754 round-to-nearest-even fp32 -> fp16 (the build's default cast; no reference
 * counterpart). Pins: numpy astype(float16) over random and special values. */
uint16_t orc_f32_to_f16_rne(float f);
void orc_cast_f32_f16(const float *in, uint16_t *out, size_t n, int rtz);
void orc_cast_f16_f32(const uint16_t *in, float *out, size_t n);

/* ---- COO -> CSR ---------------------------------------------------------- */
/* Restates NewSparseTensorCOO validation (tensor/sparse-tensor.go:54-73) and
 * ConvertToCSR (:127-181): triplets sorted by (row, col), duplicates kept adjacent
 * (this restatement sorts stably, the reference's sort.Slice leaves tie order
 * unspecified), RowPtr filled by the forward sweep :161-177.
 * Returns 0 on success, -1 length/shape error, -2 row out of range, -3 col out of range.
 * Pins: numpy lexsort (stable) + bincount/cumsum. */
int orc_coo_to_csr(long rows, long cols, long nnz, const int32_t *ri, const int32_t *ci,
                   const float *v, int32_t *rowptr, int32_t *idx, float *data);
/* Restates SparseTensor.ToDense for CSR (tensor/sparse-tensor.go:251-258) and
 * perform_sparse_to_dense (metal_bridge_sparse.m:366-377): last duplicate written wins. */
void orc_csr_to_dense(long rows, long cols, const int32_t *rowptr, const int32_t *idx,
                      const float *data, float *out);

/* ---- SpMM / SpMV --------------------------------------------------------- */
/* Restates perform_sparse_dense_matmul, internal/cgo/metal_bridge_sparse.m:117-133:
 * C = 0; for i, for k in [rp[i],rp[i+1]), for j<N: C[i,j] += v[k]*D[col[k],j], fp32,
 * CSR order. fma=1 rounds each update once (fmaf), fma=0 rounds product and sum
 * separately. Pins: scipy.sparse float64 product, dense GEMM of ToDense. */
void orc_spmm_csr_f32(long M, long N, const int32_t *rowptr, const int32_t *col,
                      const float *val, const float *D, long ldd, float *C, long ldc, int fma);
/* Same loop in float64 (the accuracy reference). */
/* Row-parallel forms of the two loops above (bit-identical results; CPU baseline only). */
void orc_spmm_csr_f32_par(long M, long N, const int32_t *rowptr, const int32_t *col, const float *val,
                          const float *D, long ldd, float *C, long ldc, int use_fma, int threads);
void orc_spmv_csr_f32_par(long M, const int32_t *rowptr, const int32_t *col, const float *val, const float *x,
                          float *y, int use_fma, int threads);
void orc_spmm_csr_f64(long M, long N, const int32_t *rowptr, const int32_t *col,
                      const float *val, const float *D, long ldd, double *C, long ldc, int threads);
/* Restates perform_sparse_matvec, metal_bridge_sparse.m:325-339: y[i] = sequential
 * fp32 sum of v[k]*x[col[k]]. */
void orc_spmv_csr_f32(long M, const int32_t *rowptr, const int32_t *col, const float *val,
                      const float *x, float *y, int fma);
void orc_spmv_csr_f64(long M, const int32_t *rowptr, const int32_t *col, const float *val,
                      const float *x, double *y);

/* ---- remaining sparse entry points ---------------------------------------- */
/* Restates perform_sparse_sparse_matmul, metal_bridge_sparse.m:49-84: C = 0; for each
 * (i, j) merge A's CSR row i with B's CSC column j, equal indices pair up and both
 * advance, sum += a*b (fma=1: fmaf); store only a nonzero sum. Pins: equals the float64
 * dense product of ToDense(A) and ToDense(B) for distinct sorted indices; brute force on
 * tiny shapes; a hand-worked duplicate-pairing case. */
void orc_spgemm_csr_csc_f32(long M, long N, const int32_t *arp, const int32_t *acol, const float *aval,
                            const int32_t *bcp, const int32_t *brow, const float *bval, float *C, long ldc, int fma);
/* Restates perform_dense_sparse_matmul, metal_bridge_sparse.m:160-176: C = 0; for each
 * column j of the CSC B, for each entry k, for each row i: C[i,j] += A[i,row_k]*v_k
 * (fma=1: fmaf). Pins: numpy float64 A @ ToDense(B). */
void orc_dense_csc_f32(long M, long K, long N, const float *A, long lda, const int32_t *bcp, const int32_t *brow,
                       const float *bval, float *C, long ldc, int fma);
/* Restates perform_sparse_add, metal_bridge_sparse.m:212-266: per row, merge the two
 * CSR rows by column (INT_MAX marks an exhausted row); equal columns are added and
 * dropped when the sum is 0; the others are copied. Writes COO triplets in that order.
 * Returns 0, or -2 (and stops) once max_nnz would be exceeded. *actual = count.
 * Pins: ToDense(A) + ToDense(B) equals the COO result scattered; hand-worked merge cases
 * (cancellation, one-sided entries, empty rows). */
int orc_sparse_add(long M, const int32_t *arp, const int32_t *acol, const float *aval, const int32_t *brp,
                   const int32_t *bcol, const float *bval, int32_t *ri, int32_t *ci, float *vv, long max_nnz,
                   long *actual);
/* Restates perform_dense_to_sparse, metal_bridge_sparse.m:403-424: row-major scan,
 * keep fabsf(v) > threshold. Returns 0 or -2 past max_nnz. Pins: numpy nonzero of
 * |D| > threshold (row-major order). */
int orc_dense_to_coo(long M, long N, const float *D, float threshold, int32_t *ri, int32_t *ci, float *vv,
                     long max_nnz, long *actual);

/* ---- activations / fused linear ----------------------------------------- */
/* Activation codes follow the Go ActivationType enum, gpu/matrix/activation.go:20-29:
 * 0 ReLU, 1 Sigmoid, 2 Tanh, 3 Softmax (not element-wise: rejected), 4 LeakyReLU,
 * 5 ELU, 6 Swish, 7 GELU (tanh form); -1 identity (no activation; build extension).
 * Formulas: ReLU metal_bridge_activation.m:46, Sigmoid :104-106, Tanh :167,
 * LeakyReLU :393, ELU :455-463, Swish :535-538, GELU :629-634 (inner clamped to +-88).
 * Pins: ReLU vector gpu/matrix/activation_test.go:32-51, GELU(0)=0 :282-285,
 * closed forms (tanh(0)=0, sigmoid(0)=1/2, large-|x| limits). Returns NaN for code 3. */
double orc_act_f64(int code, double alpha, double x);
float orc_act_f32(int code, float alpha, float x);
/* Row-wise softmax (ActivationForward Softmax, metal_bridge_activation.m:206-242,
 * :283-325) in float64. Pinned by tests/test_oracle.py: rows sum to 1, invariance to a
 * per-row shift, the two-element closed form 1/(1+exp(b-a)), scipy.special.softmax. */
void orc_softmax_rows_f64(long rows, long cols, const float *in, double *out);
/* Y[b,o] = act(sum_i X[b,i]*W(i,o) + bias[o]) in float64; W(i,o) = W[i*out+o] when
 * w_out_in=0 (reference layout, fused-operations.go:413-415 / default.metal:478) or
 * W[o*in+i] when w_out_in=1 (nn.Linear layout). bias may be NULL. */
void orc_linear_f64(long batch, long in, long out, const float *X, const float *W, int w_out_in,
                    const float *bias, int act, double alpha, double *Y, int threads);

/* d act(x)/dx at x, float64, for the codes above (-1 gives 1). The derivatives of the
 * formulas of orc_act_f64: ReLU [x>0]; Sigmoid s(1-s); Tanh 1-t^2; LeakyReLU x>0 ? 1 : a;
 * ELU x>0 ? 1 : a*e^x; Swish s + c*s*(1-s) at c = clamp(x); GELU
 * 0.5(1+t) + 0.5x(1-t^2)*sqrt(2/pi)(1+3*0.044715x^2), t = tanh(clamped inner) (the
 * derivative expression of metal_bridge_activation.m:689-697 at the input x).
 * The reference's FusedLinearActivation.Backward (fused-operations.go:486-523) hands
 * the PRE-activation to helpers whose formulas expect the activation OUTPUT
 * (metal_bridge_activation.m:131-134, :192-195, :667-698); for ReLU and LeakyReLU the
 * two agree, for Sigmoid, Tanh and GELU this restatement follows the mathematics
 * (derivative at the input), which the build implements. Pins: central finite
 * differences of orc_act_f64 (tests/test_oracle.py) and closed forms (GELU'(0) = 1/2,
 * sigmoid'(0) = 1/4, tanh'(0) = 1, Swish'(0) = 1/2). */
double orc_act_grad_f64(int code, double alpha, double x);
/* g[i] = dy[i] * orc_act_grad_f64(code, alpha, pre[i]) * scale, i < n. */
void orc_act_backward_f64(int code, double alpha, double scale, const float *dy, const float *pre, long n,
                          double *g);

/* ---- activation backward from the activation OUTPUT (reference bridge) ------ */
/* Restates perform_activation_*_backward, internal/cgo/metal_bridge_activation.m, which take
 * the gradient g and the activation's OUTPUT y (gpu/matrix/activation.go:177-300), in fp32
 * with one rounding per operation as the C source is written (this file is built with
 * -ffp-contract=off): ReLU y>0 ? g : 0 (:77-79); Sigmoid g*y*(1-y) (:137-140); Tanh
 * g*(1-y*y) (:198-201); LeakyReLU g*(y>0 ? 1 : a) (:425-429); ELU g*(y>0 ? 1 : y+a)
 * (:494-506); Swish: |y|<1e-8 -> g*0.5, else x from y by three Newton steps on
 * x*sigmoid(x) = y starting at x = y (a step is skipped when |f'| <= 1e-8), then
 * g*(s + x*s*(1-s)) (:569-599); GELU: three Newton steps on GELU(x) = y from x = y, inner
 * argument clamped to +-88, then g*GELU'(x) (:665-697). Other codes return g.
 * Pins (tests/test_oracle.py): for y = act(x) computed in float64, the result equals
 * g*act'(x) from the finite-difference-pinned orc_act_grad_f64 (the reference's formulas
 * are exact identities for Sigmoid, Tanh, ELU, LeakyReLU, ReLU; for Swish and GELU where the
 * three Newton steps converge); the special cases Swish(|y|<1e-8) = g/2 and GELU(y=0) =
 * g/2. */
float orc_act_backward_out_f32(int code, float alpha, float g, float y);
void orc_act_backward_out_array_f32(int code, float alpha, const float *g, const float *y, float *out, long n);
/* Restates perform_activation_softmax_{1d,2d}_backward (:247-281, :329-369): per row,
 * dot = sequential fp32 sum of g*y, then out = y*(g - dot). Pins: float64 central finite
 * differences of x -> sum(g * softmax(x)) at y = softmax(x). */
void orc_softmax_backward_f32(long rows, long cols, const float *g, const float *y, float *out);

/* ---- transpose ----------------------------------------------------------- */
/* out[j,i] = in[i,j]; restates metal_bridge_matrix.m:162-166. */
void orc_transpose_f32(long rows, long cols, const float *in, float *out);

/* ---- error metric -------------------------------------------------------- */
/* ||X - R||_F / ||R||_F with X fp32 and R float64 (||R||=0 -> returns ||X||_F). */
double orc_rel_frob(const float *X, const double *R, size_t n);

#ifdef __cplusplus
}
#endif
#endif
