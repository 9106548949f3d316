/*
 * oracle.c — CPU checker for the GEMM / fp16 / CSR / SpMM / SpMV path.
 *
 * TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py. The product library never links it.
 *
 * Built with -ffp-contract=off so that every a*b+c written below rounds twice
 * unless fmaf()/fma() is called explicitly.
 */
#include "oracle.h"

#include <limits.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------- */
/* synthetic data                                                            */
/* ------------------------------------------------------------------------- */
static inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

uint64_t orc_splitmix64(uint64_t seed, uint64_t stream, uint64_t i) {
  uint64_t base = seed ^ mix64(stream + 0x632BE59BD9B4E019ULL);
  return mix64(base + (i + 1) * 0x9E3779B97F4A7C15ULL);
}

void orc_fill_uniform_f32(float *out, size_t n, uint64_t seed, uint64_t stream, float lo, float hi) {
  const double scale = 1.0 / 16777216.0; /* 2^-24 */
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < (long long)n; ++i) {
    double u = (double)(orc_splitmix64(seed, stream, (uint64_t)i) >> 40) * scale;
    out[i] = (float)((double)lo + ((double)hi - (double)lo) * u);
  }
}

void orc_fill_normal_f32(float *out, size_t n, uint64_t seed, uint64_t stream, float mean, float stddev) {
  const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < (long long)n; ++i) {
    uint64_t a = orc_splitmix64(seed, stream, 2 * (uint64_t)i);
    uint64_t b = orc_splitmix64(seed, stream, 2 * (uint64_t)i + 1);
    double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0); /* (0,1] */
    double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);         /* [0,1) */
    double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
    out[i] = (float)((double)mean + (double)stddev * z);
  }
}

/* ------------------------------------------------------------------------- */
/* float64 GEMM                                                              */
/* ------------------------------------------------------------------------- */
static inline double elemA(int tA, const float *A, long lda, long i, long k) {
  return tA ? (double)A[k * lda + i] : (double)A[i * lda + k];
}

/* Computes rows [r0,r1) of op(A)*op(B) into acc rows (double, ldc=N). op(B) is
 * first widened row-panel by row-panel into a K-contiguous double buffer so the
 * inner loop is a unit-stride dot product regardless of transB. */
static void gemm_rows_f64(int tA, int tB, long N, long K, const float *A, long lda, const float *B,
                          long ldb, const long *rowlist, long nrows, double *C, long ldc,
                          double alpha, double beta, int threads) {
  /* Bt[j*K + k] = op(B)[k][j] */
  double *Bt = (double *)malloc(sizeof(double) * (size_t)N * (size_t)K);
  if (!Bt) return;
#pragma omp parallel for schedule(static) num_threads(threads)
  for (long j = 0; j < N; ++j)
    for (long k = 0; k < K; ++k)
      Bt[(size_t)j * K + k] = tB ? (double)B[j * ldb + k] : (double)B[k * ldb + j];

#pragma omp parallel num_threads(threads)
  {
    double *arow = (double *)malloc(sizeof(double) * (size_t)K);
#pragma omp for schedule(dynamic, 4)
    for (long r = 0; r < nrows; ++r) {
      long i = rowlist ? rowlist[r] : r;
      for (long k = 0; k < K; ++k) arow[k] = elemA(tA, A, lda, i, k);
      double *crow = C + (size_t)r * ldc;
      for (long j = 0; j < N; ++j) {
        const double *bcol = Bt + (size_t)j * K;
        double s0 = 0, s1 = 0, s2 = 0, s3 = 0;
        long k = 0;
        for (; k + 4 <= K; k += 4) {
          s0 += arow[k] * bcol[k];
          s1 += arow[k + 1] * bcol[k + 1];
          s2 += arow[k + 2] * bcol[k + 2];
          s3 += arow[k + 3] * bcol[k + 3];
        }
        for (; k < K; ++k) s0 += arow[k] * bcol[k];
        double s = (s0 + s1) + (s2 + s3);
        crow[j] = (beta == 0.0) ? alpha * s : alpha * s + beta * crow[j];
      }
    }
    free(arow);
  }
  free(Bt);
}

void orc_gemm_f64(int transA, int transB, long M, long N, long K, double alpha, const float *A,
                  long lda, const float *B, long ldb, double beta, double *C, long ldc, int threads) {
  if (threads <= 0) threads = 1;
  if (K == 0) {
    for (long i = 0; i < M; ++i)
      for (long j = 0; j < N; ++j) C[i * ldc + j] = (beta == 0.0) ? 0.0 : beta * C[i * ldc + j];
    return;
  }
  gemm_rows_f64(transA, transB, N, K, A, lda, B, ldb, NULL, M, C, ldc, alpha, beta, threads);
}

void orc_gemm_f64_rows(int transA, int transB, long M, long N, long K, const float *A, long lda,
                       const float *B, long ldb, const long *rows, long nrows, double *C, long ldc,
                       int threads) {
  (void)M;
  if (threads <= 0) threads = 1;
  gemm_rows_f64(transA, transB, N, K, A, lda, B, ldb, rows, nrows, C, ldc, 1.0, 0.0, threads);
}

/* ------------------------------------------------------------------------- */
/* fp16                                                                      */
/* ------------------------------------------------------------------------- */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* mixed-precision.go:106-151, statement by statement. */
uint16_t orc_f32_to_f16_rtz(float f) {
  uint32_t bits = f2u(f);
  uint32_t sign = (bits >> 31) & 0x1u;
  uint32_t exp = (bits >> 23) & 0xFFu;
  uint32_t mant = bits & 0x7FFFFFu;
  if (exp == 0) return (uint16_t)(sign << 15);                 /* :115-117 */
  if (exp == 0xFF) {                                           /* :118-127 */
    if (mant == 0) return (uint16_t)((sign << 15) | 0x7C00u);
    return (uint16_t)((sign << 15) | 0x7C00u | (mant >> 13));
  }
  int32_t e = (int32_t)exp - 127 + 15;                         /* :130 */
  if (e >= 31) return (uint16_t)((sign << 15) | 0x7C00u);      /* :132-134 */
  if (e <= 0) {                                                /* :135-147 */
    if (e < -10) return (uint16_t)(sign << 15);
    uint32_t shift = (uint32_t)(1 - e);
    mant = (mant | 0x800000u) >> shift;
    return (uint16_t)((sign << 15) | (mant >> 13));
  }
  return (uint16_t)((sign << 15) | ((uint32_t)e << 10) | (mant >> 13)); /* :150 */
}

/* mixed-precision.go:154-189. */
float orc_f16_to_f32(uint16_t h) {
  uint32_t bits = h;
  uint32_t sign = (bits >> 15) & 0x1u;
  uint32_t exp = (bits >> 10) & 0x1Fu;
  uint32_t mant = bits & 0x3FFu;
  uint32_t r;
  if (exp == 0) {
    if (mant == 0) {
      r = sign << 31;
    } else {
      while ((mant & 0x400u) == 0) { mant <<= 1; exp--; } /* uint32 wrap, as in Go */
      mant &= 0x3FFu;
      exp = exp - 15 + 127 + 1;
      r = (sign << 31) | (exp << 23) | (mant << 13);
    }
  } else if (exp == 31) {
    r = (sign << 31) | 0x7F800000u | (mant << 13);
  } else {
    exp = exp - 15 + 127;
    r = (sign << 31) | (exp << 23) | (mant << 13);
  }
  return u2f(r);
}

/* IEEE 754 binary32 -> binary16, round to nearest, ties to even; NaN stays NaN (quiet). */
uint16_t orc_f32_to_f16_rne(float f) {
  uint32_t x = f2u(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) { /* inf / nan */
    if (ax == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
  }
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
  if (ax < 0x38800000u) {                                    /* below 2^-14: subnormal or zero */
    if (ax < 0x33000000u) return (uint16_t)sign;             /* < 2^-25: rounds to 0 (2^-25 ties to 0) */
    uint32_t e = ax >> 23;                                   /* 102..112 */
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126 - e;                                /* value = m * 2^(e-150); unit 2^-24 */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t e = (ax >> 23) - 127 + 15;
  uint32_t m = ax & 0x7FFFFFu;
  uint32_t q = (e << 10) | (m >> 13);
  uint32_t rem = m & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
  return (uint16_t)(sign | q);
}

void orc_cast_f32_f16(const float *in, uint16_t *out, size_t n, int rtz) {
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < (long long)n; ++i)
    out[i] = rtz ? orc_f32_to_f16_rtz(in[i]) : orc_f32_to_f16_rne(in[i]);
}

void orc_cast_f16_f32(const uint16_t *in, float *out, size_t n) {
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < (long long)n; ++i) out[i] = orc_f16_to_f32(in[i]);
}

/* ------------------------------------------------------------------------- */
/* COO -> CSR                                                                */
/* ------------------------------------------------------------------------- */
int orc_coo_to_csr(long rows, long cols, long nnz, const int32_t *ri, const int32_t *ci,
                   const float *v, int32_t *rowptr, int32_t *idx, float *data) {
  if (rows < 0 || cols < 0 || nnz < 0) return -1;
  for (long k = 0; k < nnz; ++k) { /* sparse-tensor.go:66-73 */
    if (ri[k] < 0 || ri[k] >= rows) return -2;
    if (ci[k] < 0 || ci[k] >= cols) return -3;
  }
  /* Stable order by (row, col): counting sort by row (stable), then a stable
   * insertion sort of the columns inside each row (rows average tens of entries). */
  long *cnt = (long *)calloc((size_t)rows + 1, sizeof(long));
  long *perm = (long *)malloc(sizeof(long) * (size_t)(nnz > 0 ? nnz : 1));
  if (!cnt || !perm) { free(cnt); free(perm); return -1; }
  for (long k = 0; k < nnz; ++k) cnt[ri[k] + 1]++;
  for (long r = 0; r < rows; ++r) cnt[r + 1] += cnt[r];
  for (long r = 0; r <= rows; ++r) rowptr[r] = (int32_t)cnt[r];
  for (long k = 0; k < nnz; ++k) perm[cnt[ri[k]]++] = k;
  for (long r = 0; r < rows; ++r) {
    long s = rowptr[r], e = rowptr[r + 1];
    for (long a = s + 1; a < e; ++a) {
      long p = perm[a];
      long b = a - 1;
      while (b >= s && ci[perm[b]] > ci[p]) { perm[b + 1] = perm[b]; --b; }
      perm[b + 1] = p;
    }
  }
  for (long k = 0; k < nnz; ++k) { idx[k] = ci[perm[k]]; data[k] = v[perm[k]]; }
  free(cnt);
  free(perm);
  return 0;
}

void orc_csr_to_dense(long rows, long cols, const int32_t *rowptr, const int32_t *idx,
                      const float *data, float *out) {
  memset(out, 0, sizeof(float) * (size_t)rows * (size_t)cols);
  for (long r = 0; r < rows; ++r)
    for (long k = rowptr[r]; k < rowptr[r + 1]; ++k) out[r * cols + idx[k]] = data[k];
}

/* ------------------------------------------------------------------------- */
/* SpMM / SpMV                                                               */
/* ------------------------------------------------------------------------- */
void orc_spmm_csr_f32(long M, long N, const int32_t *rowptr, const int32_t *col, const float *val,
                      const float *D, long ldd, float *C, long ldc, int use_fma) {
  for (long i = 0; i < M; ++i)
    for (long j = 0; j < N; ++j) C[i * ldc + j] = 0.0f; /* metal_bridge_sparse.m:117 */
  for (long i = 0; i < M; ++i) {                         /* :120-133 */
    long start = rowptr[i], end = rowptr[i + 1];
    for (long k = start; k < end; ++k) {
      int c = col[k];
      float a = val[k];
      const float *drow = D + (long)c * ldd;
      float *crow = C + i * ldc;
      if (use_fma) {
        for (long j = 0; j < N; ++j) crow[j] = fmaf(a, drow[j], crow[j]);
      } else {
        for (long j = 0; j < N; ++j) { float p = a * drow[j]; crow[j] = crow[j] + p; }
      }
    }
  }
}

/* The same loops with the rows split over `threads` OpenMP threads: each row is computed
 * exactly as in orc_spmm_csr_f32 / orc_spmv_csr_f32, so the results are bit-identical.
 * The CPU baseline's parallel line (the reference runs them on one thread). */
void orc_spmm_csr_f32_par(long M, long N, const int32_t *rowptr, const int32_t *col, const float *val,
                          const float *D, long ldd, float *C, long ldc, int use_fma, int threads) {
  if (threads <= 0) threads = 1;
#pragma omp parallel for schedule(dynamic, 64) num_threads(threads)
  for (long i = 0; i < M; ++i) {
    float *crow = C + i * ldc;
    for (long j = 0; j < N; ++j) crow[j] = 0.0f;
    for (long k = rowptr[i]; k < rowptr[i + 1]; ++k) {
      const float a = val[k];
      const float *drow = D + (long)col[k] * ldd;
      if (use_fma) {
        for (long j = 0; j < N; ++j) crow[j] = fmaf(a, drow[j], crow[j]);
      } else {
        for (long j = 0; j < N; ++j) { float p = a * drow[j]; crow[j] = crow[j] + p; }
      }
    }
  }
}

void orc_spmv_csr_f32_par(long M, const int32_t *rowptr, const int32_t *col, const float *val, const float *x,
                          float *y, int use_fma, int threads) {
  if (threads <= 0) threads = 1;
#pragma omp parallel for schedule(dynamic, 256) num_threads(threads)
  for (long i = 0; i < M; ++i) {
    float sum = 0.0f;
    for (long k = rowptr[i]; k < rowptr[i + 1]; ++k) {
      if (use_fma) sum = fmaf(val[k], x[col[k]], sum);
      else { float p = val[k] * x[col[k]]; sum = sum + p; }
    }
    y[i] = sum;
  }
}

void orc_spmm_csr_f64(long M, long N, const int32_t *rowptr, const int32_t *col, const float *val,
                      const float *D, long ldd, double *C, long ldc, int threads) {
  if (threads <= 0) threads = 1;
#pragma omp parallel for schedule(dynamic, 64) num_threads(threads)
  for (long i = 0; i < M; ++i) {
    double *crow = C + i * ldc;
    for (long j = 0; j < N; ++j) crow[j] = 0.0;
    for (long k = rowptr[i]; k < rowptr[i + 1]; ++k) {
      double a = val[k];
      const float *drow = D + (long)col[k] * ldd;
      for (long j = 0; j < N; ++j) crow[j] += a * (double)drow[j];
    }
  }
}

void orc_spmv_csr_f32(long M, const int32_t *rowptr, const int32_t *col, const float *val,
                      const float *x, float *y, int use_fma) {
  for (long i = 0; i < M; ++i) { /* metal_bridge_sparse.m:328-338 */
    float sum = 0.0f;
    for (long k = rowptr[i]; k < rowptr[i + 1]; ++k) {
      if (use_fma) sum = fmaf(val[k], x[col[k]], sum);
      else { float p = val[k] * x[col[k]]; sum = sum + p; }
    }
    y[i] = sum;
  }
}

void orc_spmv_csr_f64(long M, const int32_t *rowptr, const int32_t *col, const float *val,
                      const float *x, double *y) {
  for (long i = 0; i < M; ++i) {
    double s = 0.0;
    for (long k = rowptr[i]; k < rowptr[i + 1]; ++k) s += (double)val[k] * (double)x[col[k]];
    y[i] = s;
  }
}

/* ------------------------------------------------------------------------- */
/* remaining sparse entry points                                             */
/* ------------------------------------------------------------------------- */
void orc_spgemm_csr_csc_f32(long M, long N, const int32_t *arp, const int32_t *acol, const float *aval,
                            const int32_t *bcp, const int32_t *brow, const float *bval, float *C, long ldc, int fma) {
  for (long i = 0; i < M; ++i)
    for (long j = 0; j < N; ++j) C[i * ldc + j] = 0.0f; /* :50 memset */
  for (long i = 0; i < M; ++i)
    for (long j = 0; j < N; ++j) {
      long ai = arp[i], ae = arp[i + 1], bi = bcp[j], be = bcp[j + 1];
      float sum = 0.0f;
      while (ai < ae && bi < be) { /* :66-78 */
        int ac = acol[ai], br = brow[bi];
        if (ac == br) {
          sum = fma ? fmaf(aval[ai], bval[bi], sum) : sum + aval[ai] * bval[bi];
          ++ai;
          ++bi;
        } else if (ac < br) {
          ++ai;
        } else {
          ++bi;
        }
      }
      if (sum != 0.0f) C[i * ldc + j] = sum; /* :80-82 */
    }
}

void orc_dense_csc_f32(long M, long K, long N, const float *A, long lda, const int32_t *bcp, const int32_t *brow,
                       const float *bval, float *C, long ldc, int fma) {
  (void)K;
  for (long i = 0; i < M; ++i)
    for (long j = 0; j < N; ++j) C[i * ldc + j] = 0.0f; /* :161 */
  for (long j = 0; j < N; ++j)                          /* :164-176 */
    for (long k = bcp[j]; k < bcp[j + 1]; ++k) {
      const int r = brow[k];
      const float v = bval[k];
      for (long i = 0; i < M; ++i) {
        float *c = C + i * ldc + j;
        *c = fma ? fmaf(A[i * lda + r], v, *c) : *c + A[i * lda + r] * v;
      }
    }
}

int orc_sparse_add(long M, const int32_t *arp, const int32_t *acol, const float *aval, const int32_t *brp,
                   const int32_t *bcol, const float *bval, int32_t *ri, int32_t *ci, float *vv, long max_nnz,
                   long *actual) {
  long n = 0;
  for (long i = 0; i < M; ++i) { /* :214-259 */
    long ai = arp[i], ae = arp[i + 1], bi = brp[i], be = brp[i + 1];
    while (ai < ae || bi < be) {
      if (n >= max_nnz) {
        *actual = n;
        return -2;
      }
      int ac = ai < ae ? acol[ai] : INT_MAX, bc = bi < be ? bcol[bi] : INT_MAX;
      if (ac == bc && ac != INT_MAX) {
        float sum = aval[ai] + bval[bi];
        if (sum != 0.0f) {
          ri[n] = (int32_t)i;
          ci[n] = ac;
          vv[n] = sum;
          ++n;
        }
        ++ai;
        ++bi;
      } else if (ac < bc) {
        ri[n] = (int32_t)i;
        ci[n] = ac;
        vv[n] = aval[ai];
        ++n;
        ++ai;
      } else {
        ri[n] = (int32_t)i;
        ci[n] = bc;
        vv[n] = bval[bi];
        ++n;
        ++bi;
      }
    }
  }
  *actual = n;
  return 0;
}

int orc_dense_to_coo(long M, long N, const float *D, float threshold, int32_t *ri, int32_t *ci, float *vv,
                     long max_nnz, long *actual) {
  long n = 0;
  for (long i = 0; i < M; ++i) /* :407-423 */
    for (long j = 0; j < N; ++j) {
      const float v = D[i * N + j];
      if (fabsf(v) > threshold) {
        if (n >= max_nnz) {
          *actual = n;
          return -2;
        }
        ri[n] = (int32_t)i;
        ci[n] = (int32_t)j;
        vv[n] = v;
        ++n;
      }
    }
  *actual = n;
  return 0;
}

/* ------------------------------------------------------------------------- */
/* activations / linear                                                      */
/* ------------------------------------------------------------------------- */
static inline double clampd(double x, double lo, double hi) { return x < lo ? lo : (x > hi ? hi : x); }

double orc_act_f64(int code, double alpha, double x) {
  switch (code) {
    case -1: return x;
    case 0: return x > 0.0 ? x : 0.0;                                         /* fmaxf(0,x) */
    case 1: { double c = clampd(x, -88.0, 88.0); return 1.0 / (1.0 + exp(-c)); }
    case 2: return tanh(x);
    case 4: return x > 0.0 ? x : alpha * x;
    case 5: return x > 0.0 ? x : alpha * (exp(x < -88.0 ? -88.0 : x) - 1.0);
    case 6: { double c = clampd(x, -88.0, 88.0); return c / (1.0 + exp(-c)); }
    case 7: {
      double inner = 0.7978845608028654 * (x + 0.044715 * x * x * x);
      inner = clampd(inner, -88.0, 88.0);
      return 0.5 * x * (1.0 + tanh(inner));
    }
    default: return NAN; /* 3 = Softmax is row-wise, not an epilogue */
  }
}

float orc_act_f32(int code, float alpha, float x) {
  switch (code) {
    case -1: return x;
    case 0: return fmaxf(0.0f, x);
    case 1: { float c = fmaxf(-88.0f, fminf(88.0f, x)); return 1.0f / (1.0f + expf(-c)); }
    case 2: return tanhf(x);
    case 4: return x > 0.0f ? x : alpha * x;
    case 5: return x > 0.0f ? x : alpha * (expf(fmaxf(-88.0f, x)) - 1.0f);
    case 6: { float c = fmaxf(-88.0f, fminf(88.0f, x)); float s = 1.0f / (1.0f + expf(-c)); return c * s; }
    case 7: {
      float x3 = x * x * x;
      float inner = 0.7978845608028654f * (x + 0.044715f * x3);
      inner = fmaxf(-88.0f, fminf(88.0f, inner));
      return 0.5f * x * (1.0f + tanhf(inner));
    }
    default: return NAN;
  }
}

double orc_act_grad_f64(int code, double alpha, double x) {
  switch (code) {
    case -1: return 1.0;
    case 0: return x > 0.0 ? 1.0 : 0.0;
    case 1: { double s = 1.0 / (1.0 + exp(-clampd(x, -88.0, 88.0))); return s * (1.0 - s); }
    case 2: { double t = tanh(x); return 1.0 - t * t; }
    case 4: return x > 0.0 ? 1.0 : alpha;
    case 5: return x > 0.0 ? 1.0 : alpha * exp(x < -88.0 ? -88.0 : x);
    case 6: {
      double c = clampd(x, -88.0, 88.0), s = 1.0 / (1.0 + exp(-c));
      return s + c * s * (1.0 - s);
    }
    case 7: {
      const double k = 0.7978845608028654, a3 = 0.044715;
      double t = tanh(clampd(k * (x + a3 * x * x * x), -88.0, 88.0));
      return 0.5 * (1.0 + t) + 0.5 * x * (1.0 - t * t) * k * (1.0 + 3.0 * a3 * x * x);
    }
    default: return NAN;
  }
}

void orc_act_backward_f64(int code, double alpha, double scale, const float *dy, const float *pre, long n,
                          double *g) {
  for (long i = 0; i < n; ++i) g[i] = (double)dy[i] * orc_act_grad_f64(code, alpha, (double)pre[i]) * scale;
}

void orc_linear_f64(long batch, long in, long out, const float *X, const float *W, int w_out_in,
                    const float *bias, int act, double alpha, double *Y, int threads) {
  /* op(B)[k][j] = W(i=k, o=j): reference layout W[in,out] is transB=0 with ldb=out;
   * nn.Linear layout W[out,in] is transB=1 with ldb=in. */
  orc_gemm_f64(0, w_out_in ? 1 : 0, batch, out, in, 1.0, X, in, W, w_out_in ? in : out, 0.0, Y, out,
               threads);
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
  for (long b = 0; b < batch; ++b)
    for (long o = 0; o < out; ++o) {
      double s = Y[b * out + o] + (bias ? (double)bias[o] : 0.0);
      Y[b * out + o] = orc_act_f64(act, alpha, s);
    }
}

/* Row-wise softmax in float64 of a [rows, cols] fp32 matrix (ActivationForward's
 * Softmax: metal_bridge_activation.m:206-242 for 1-D, :283-325 for 2-D): m = the row's
 * maximum by fmax from its first element (NaNs skipped), y = exp(x - m), then y /= sum. */
void orc_softmax_rows_f64(long rows, long cols, const float *in, double *out) {
  for (long r = 0; r < rows; ++r) {
    const float *x = in + r * cols;
    double *y = out + r * cols;
    if (cols <= 0) continue;
    double m = x[0];
    for (long i = 1; i < cols; ++i) m = fmax(m, (double)x[i]);
    double s = 0.0;
    for (long i = 0; i < cols; ++i) {
      y[i] = exp((double)x[i] - m);
      s += y[i];
    }
    for (long i = 0; i < cols; ++i) y[i] /= s;
  }
}

/* activation backward from the output: metal_bridge_activation.m:54-702 */
float orc_act_backward_out_f32(int code, float alpha, float g, float y) {
  switch (code) {
    case 0: return y > 0.0f ? g : 0.0f;
    case 1: return g * y * (1.0f - y);
    case 2: return g * (1.0f - y * y);
    case 4: return g * (y > 0.0f ? 1.0f : alpha);
    case 5: return g * (y > 0.0f ? 1.0f : y + alpha);
    case 6: {
      if (fabsf(y) < 1e-8f) return g * 0.5f;
      float x = y;
      for (int it = 0; it < 3; ++it) {
        float s = 1.0f / (1.0f + expf(-x));
        float f = x * s - y;
        float df = s + x * s * (1.0f - s);
        if (fabsf(df) > 1e-8f) x = x - f / df;
      }
      float s = 1.0f / (1.0f + expf(-x));
      return g * (s + x * s * (1.0f - s));
    }
    case 7: {
      const float k = 0.7978845608028654f, c = 0.044715f;
      float x = y;
      for (int it = 0; it < 3; ++it) {
        float x3 = x * x * x;
        float inner = k * (x + c * x3);
        inner = fmaxf(-88.0f, fminf(88.0f, inner));
        float t = tanhf(inner);
        float f = 0.5f * x * (1.0f + t) - y;
        float dt = 1.0f - t * t;
        float di = k * (1.0f + 3.0f * c * x * x);
        float df = 0.5f * (1.0f + t) + 0.5f * x * dt * di;
        if (fabsf(df) > 1e-8f) x = x - f / df;
      }
      float x3 = x * x * x;
      float inner = k * (x + c * x3);
      inner = fmaxf(-88.0f, fminf(88.0f, inner));
      float t = tanhf(inner);
      float sech2 = 1.0f - t * t;
      float di = k * (1.0f + 3.0f * c * x * x);
      return g * (0.5f * (1.0f + t) + 0.5f * x * sech2 * di);
    }
    default: return g;
  }
}

void orc_act_backward_out_array_f32(int code, float alpha, const float *g, const float *y, float *out, long n) {
  for (long i = 0; i < n; ++i) out[i] = orc_act_backward_out_f32(code, alpha, g[i], y[i]);
}

void orc_softmax_backward_f32(long rows, long cols, const float *g, const float *y, float *out) {
  for (long r = 0; r < rows; ++r) {
    const float *gr = g + r * cols, *yr = y + r * cols;
    float dot = 0.0f;
    for (long i = 0; i < cols; ++i) dot += gr[i] * yr[i];
    for (long i = 0; i < cols; ++i) out[r * cols + i] = yr[i] * (gr[i] - dot);
  }
}

/* ------------------------------------------------------------------------- */
void orc_transpose_f32(long rows, long cols, const float *in, float *out) {
  for (long i = 0; i < rows; ++i)
    for (long j = 0; j < cols; ++j) out[j * rows + i] = in[i * cols + j];
}

double orc_rel_frob(const float *X, const double *R, size_t n) {
  double num = 0.0, den = 0.0;
  for (size_t i = 0; i < n; ++i) {
    double d = (double)X[i] - R[i];
    num += d * d;
    den += R[i] * R[i];
  }
  if (den == 0.0) return sqrt(num);
  return sqrt(num / den);
}
