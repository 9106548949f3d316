// sparse_ops.hip — the remaining sparse entry points of the reference bridge, as HIP
// kernels for gfx950:
//
//   CSR x CSC -> dense      perform_sparse_sparse_matmul   (metal_bridge_sparse.m:26-91)
//   CSR + CSR -> COO        perform_sparse_add             (:186-267)
//   values *= scalar        perform_sparse_scalar_multiply (:270-294)
//   CSR -> dense            perform_sparse_to_dense        (:345-381)
//   dense -> COO            perform_dense_to_sparse        (:384-429)
//
// (Dense x CSC is CSR SpMM of the transposed problem; see bridge.cpp.) Each kernel
// follows the reference loop's order per output, so results match it bit for bit:
//  * sparse x sparse: one thread per output (i, j) runs the reference's merge of A's
//    row i with B's column j (equal indices pair up and both advance), accumulating
//    with one fma per match; a zero sum leaves the output +0 as the reference's
//    memset does;
//  * add and dense -> COO: a count pass, a host prefix sum over rows, then a write
//    pass in which each row's entries keep the reference's order (merge order, or
//    column order via a wave ballot);
//  * CSR -> dense: one thread per row writes its entries in CSR order, so a later
//    duplicate overwrites an earlier one, as in the reference.
// Index arrays are validated where they are used as addresses (flags[0]: bad row
// pointers, flags[1]: index out of range); the merges only compare indices, so they
// read nothing out of bounds whatever the values, and need only the pointer check.
#include <algorithm>
#include <climits>

#include "common.h"

namespace gn {
namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ bool ptr_pair(const int32_t *ptr, long i, long nnz, int &s, int &e) {
  s = ptr[i];
  e = ptr[i + 1];
  if (s < 0 || e < s || (long)e > nnz) {
    s = e = 0;
    return false;
  }
  return true;
}

// ------------------------------------------------------------------ CSR x CSC -> dense
__global__ void __launch_bounds__(kBlock) spgemm_merge_kernel(long M, long N, long annz, long bnnz,
                                                              const int32_t *__restrict__ arp,
                                                              const int32_t *__restrict__ acol,
                                                              const float *__restrict__ aval,
                                                              const int32_t *__restrict__ bcp,
                                                              const int32_t *__restrict__ brow,
                                                              const float *__restrict__ bval, float *__restrict__ C,
                                                              long ldc, int *flags) {
  const long j = (long)blockIdx.x * kBlock + threadIdx.x;
  const long i = blockIdx.y + (long)blockIdx.z * 65535;
  if (i >= M || j >= N) return;
  int as, ae, bs, be;
  if (!ptr_pair(arp, i, annz, as, ae) && flags) flags[0] = 1;
  if (!ptr_pair(bcp, j, bnnz, bs, be) && flags) flags[0] = 1;
  float sum = 0.0f;
  int ai = as, bi = bs;
  while (ai < ae && bi < be) {
    const int ac = acol[ai], br = brow[bi];
    if (ac == br) {
      sum = __builtin_fmaf(aval[ai], bval[bi], sum);
      ++ai;
      ++bi;
    } else if (ac < br) {
      ++ai;
    } else {
      ++bi;
    }
  }
  C[i * ldc + j] = sum != 0.0f ? sum : 0.0f;
}

// ------------------------------------------------------------------ CSR + CSR -> COO
// One thread per row runs the reference merge (:223-259). WRITE = false counts the
// row's outputs; WRITE = true stores them at out_off[i]. A column index outside
// [0, N) raises flags[1] and ends the row (so INT_MAX, the merge's end marker, can
// never be a real index and the merge never reads past a row).
template <bool WRITE>
__global__ void __launch_bounds__(kBlock) spadd_kernel(long M, long N, long annz, long bnnz,
                                                       const int32_t *__restrict__ arp,
                                                       const int32_t *__restrict__ acol,
                                                       const float *__restrict__ aval,
                                                       const int32_t *__restrict__ brp,
                                                       const int32_t *__restrict__ bcol,
                                                       const float *__restrict__ bval, long *__restrict__ count,
                                                       const long *__restrict__ out_off, int32_t *__restrict__ ri,
                                                       int32_t *__restrict__ ci, float *__restrict__ vv, int *flags) {
  const long i = (long)blockIdx.x * kBlock + threadIdx.x;
  if (i >= M) return;
  int as, ae, bs, be;
  if (!ptr_pair(arp, i, annz, as, ae) && flags) flags[0] = 1;
  if (!ptr_pair(brp, i, bnnz, bs, be) && flags) flags[0] = 1;
  long n = 0, o = WRITE ? out_off[i] : 0;
  int ai = as, bi = bs;
  while (ai < ae || bi < be) {
    const int ac = ai < ae ? acol[ai] : INT_MAX;
    const int bc = bi < be ? bcol[bi] : INT_MAX;
    if ((ai < ae && (unsigned)ac >= (unsigned long)N) || (bi < be && (unsigned)bc >= (unsigned long)N)) {
      if (flags) flags[1] = 1;
      break;
    }
    int col;
    float v;
    bool keep = true;
    if (ac == bc && ac != INT_MAX) {
      v = aval[ai] + bval[bi];
      keep = v != 0.0f;
      col = ac;
      ++ai;
      ++bi;
    } else if (ac < bc) {
      v = aval[ai];
      col = ac;
      ++ai;
    } else {
      v = bval[bi];
      col = bc;
      ++bi;
    }
    if (keep) {
      if (WRITE) {
        ri[o + n] = (int32_t)i;
        ci[o + n] = col;
        vv[o + n] = v;
      }
      ++n;
    }
  }
  if (!WRITE) count[i] = n;
}

// ------------------------------------------------------------------ scalar multiply
__global__ void __launch_bounds__(kBlock) scale_kernel(float *__restrict__ v, long n, float s) {
  for (long k = (long)blockIdx.x * kBlock + threadIdx.x; k < n; k += (long)gridDim.x * kBlock) v[k] *= s;
}

// ------------------------------------------------------------------ CSR -> dense
__global__ void __launch_bounds__(kBlock) zero_f32_kernel(float *__restrict__ p, long n) {
  for (long k = (long)blockIdx.x * kBlock + threadIdx.x; k < n; k += (long)gridDim.x * kBlock) p[k] = 0.0f;
}

__global__ void __launch_bounds__(kBlock) csr_to_dense_kernel(long M, long N, long nnz, const int32_t *__restrict__ rp,
                                                              const int32_t *__restrict__ col,
                                                              const float *__restrict__ val, float *__restrict__ D,
                                                              long ldd, int *flags) {
  const long i = (long)blockIdx.x * kBlock + threadIdx.x;
  if (i >= M) return;
  int s, e;
  if (!ptr_pair(rp, i, nnz, s, e) && flags) flags[0] = 1;
  for (int k = s; k < e; ++k) {
    const int c = col[k];
    if ((unsigned)c < (unsigned long)N) D[i * ldd + c] = val[k];
    else if (flags) flags[1] = 1;
  }
}

// ------------------------------------------------------------------ dense -> COO
// One wave per row; 64 columns per step. The predicate is the reference's
// fabsf(v) > threshold (NaN is dropped). WRITE = false counts; WRITE = true writes in
// column order, each lane's slot given by the number of set ballot bits below it.
template <bool WRITE>
__global__ void __launch_bounds__(kBlock) dense_to_coo_kernel(long M, long N, const float *__restrict__ D, float thr,
                                                              long *__restrict__ count, const long *__restrict__ out_off,
                                                              int32_t *__restrict__ ri, int32_t *__restrict__ ci,
                                                              float *__restrict__ vv) {
  const long i = (long)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (i >= M) return;
  long o = WRITE ? out_off[i] : 0;
  long n = 0;
  for (long c0 = 0; c0 < N; c0 += 64) {
    const long c = c0 + lane;
    const float v = c < N ? D[i * N + c] : 0.0f;
    const bool keep = c < N && fabsf(v) > thr;
    const unsigned long long m = __ballot(keep);
    if (WRITE && keep) {
      const long pos = o + n + __popcll(m & ((1ull << lane) - 1ull));
      ri[pos] = (int32_t)i;
      ci[pos] = (int32_t)c;
      vv[pos] = v;
    }
    n += __popcll(m);
  }
  if (!WRITE && lane == 0) count[i] = n;
}

unsigned grid1(long n) {
  long g = (n + kBlock - 1) / kBlock;
  if (g < 1) g = 1;
  if (g > 256L * 64) g = 256L * 64;  // grid-stride beyond
  return (unsigned)g;
}

hipError_t last() { return hipGetLastError(); }

}  // namespace

int launch_spgemm_csr_csc(long M, long N, long annz, long bnnz, const int32_t *arp, const int32_t *acol,
                          const float *aval, const int32_t *bcp, const int32_t *brow, const float *bval, float *C,
                          long ldc, int *flags, hipStream_t s, CError *err) {
  if (M < 0 || N < 0 || annz < 0 || bnnz < 0) return set_error(err, -1, "sparse-sparse: negative size");
  if (M == 0 || N == 0) return 0;
  if (!arp || !bcp || !C || (annz > 0 && (!acol || !aval)) || (bnnz > 0 && (!brow || !bval)))
    return set_error(err, -1, "sparse-sparse: NULL pointer");
  if (annz > 0x7FFFFFFFL || bnnz > 0x7FFFFFFFL) return set_error(err, -1, "sparse-sparse: exceeds int32 indexing");
  const long gx = (N + kBlock - 1) / kBlock, gz = (M + 65534) / 65535;
  if (gx > 0x7FFFFFFFL || gz > 65535) return set_error(err, -1, "sparse-sparse: result too large for the grid");
  hipLaunchKernelGGL(spgemm_merge_kernel, dim3((unsigned)gx, (unsigned)std::min(M, 65535L), (unsigned)gz),
                     dim3(kBlock), 0, s, M, N, annz, bnnz, arp, acol, aval, bcp, brow, bval, C, ldc, flags);
  hipError_t e = last();
  return e == hipSuccess ? 0 : hip_error(err, -6, "sparse-sparse launch", e);
}

int launch_spadd(bool write, long M, long N, long annz, long bnnz, const int32_t *arp, const int32_t *acol,
                 const float *aval, const int32_t *brp, const int32_t *bcol, const float *bval, long *count,
                 const long *out_off, int32_t *ri, int32_t *ci, float *vv, int *flags, hipStream_t s, CError *err) {
  if (M <= 0) return 0;
  const unsigned g = (unsigned)((M + kBlock - 1) / kBlock);
  if (write)
    hipLaunchKernelGGL(spadd_kernel<true>, dim3(g), dim3(kBlock), 0, s, M, N, annz, bnnz, arp, acol, aval, brp, bcol,
                       bval, count, out_off, ri, ci, vv, flags);
  else
    hipLaunchKernelGGL(spadd_kernel<false>, dim3(g), dim3(kBlock), 0, s, M, N, annz, bnnz, arp, acol, aval, brp, bcol,
                       bval, count, out_off, ri, ci, vv, flags);
  hipError_t e = last();
  return e == hipSuccess ? 0 : hip_error(err, -6, "sparse add launch", e);
}

int launch_scale_f32(float *v, long n, float scalar, hipStream_t s, CError *err) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(scale_kernel, dim3(grid1(n)), dim3(kBlock), 0, s, v, n, scalar);
  hipError_t e = last();
  return e == hipSuccess ? 0 : hip_error(err, -6, "scalar multiply launch", e);
}

int launch_csr_to_dense(long M, long N, long nnz, const int32_t *rp, const int32_t *col, const float *val, float *D,
                        int *flags, hipStream_t s, CError *err) {
  if (M <= 0 || N <= 0) return 0;
  hipLaunchKernelGGL(zero_f32_kernel, dim3(grid1(M * N)), dim3(kBlock), 0, s, D, M * N);
  hipLaunchKernelGGL(csr_to_dense_kernel, dim3((unsigned)((M + kBlock - 1) / kBlock)), dim3(kBlock), 0, s, M, N, nnz,
                     rp, col, val, D, N, flags);
  hipError_t e = last();
  return e == hipSuccess ? 0 : hip_error(err, -6, "sparse to dense launch", e);
}

int launch_dense_to_coo(bool write, long M, long N, const float *D, float thr, long *count, const long *out_off,
                        int32_t *ri, int32_t *ci, float *vv, hipStream_t s, CError *err) {
  if (M <= 0) return 0;
  const unsigned g = (unsigned)((M + kBlock / 64 - 1) / (kBlock / 64));
  if (write)
    hipLaunchKernelGGL(dense_to_coo_kernel<true>, dim3(g), dim3(kBlock), 0, s, M, N, D, thr, count, out_off, ri, ci,
                       vv);
  else
    hipLaunchKernelGGL(dense_to_coo_kernel<false>, dim3(g), dim3(kBlock), 0, s, M, N, D, thr, count, out_off, ri, ci,
                       vv);
  hipError_t e = last();
  return e == hipSuccess ? 0 : hip_error(err, -6, "dense to sparse launch", e);
}

}  // namespace gn
