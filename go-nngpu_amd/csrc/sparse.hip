// sparse.hip — CSR x dense SpMM and CSR SpMV for gfx950.
//
// Replaces the reference's single-threaded CPU loops perform_sparse_dense_matmul
// (internal/cgo/metal_bridge_sparse.m:117-133) and perform_sparse_matvec (:325-339).
//
// SpMM: with 16-byte aligned rows and N >= 32, spmm_band_kernel splits the columns into
// 32-float bands (one 128-byte line of a D row) and runs the bands one after another, so
// the D lines gathered at any time fit the L2 far better than whole 1 KiB D rows do: the
// kernel is bound by L2 refills from the Infinity Cache, and banding cuts them by a
// quarter at N = 256. From 65536 entries up, spmm_band_half_kernel does the same in two
// launches, each row's entries split at its first column >= K/2 (at the midpoint of its
// entries under graph capture); the partial sum goes through C. That halves the D rows each
// launch gathers from when columns are sorted and cuts the refills by another quarter. Narrower or unaligned products use a group of LPR lanes per CSR
// row, lane l accumulating columns 4l..4l+3 (or column l). Each output is accumulated in
// CSR order with one fma per entry, which reproduces the reference loop's summation
// order exactly (bit-identical to an fmaf restatement of it, in every kernel).
// Row pointers and column indices are validated in the kernel:
// an invalid row pointer pair empties the row and raises flags[0]; an out-of-range
// column skips that entry and raises flags[1]. No access ever leaves its array.
//
// SpMV: LPR lanes per row stride over the row's entries and combine their partial
// sums with an xor-shuffle tree (a different, tolerance-level summation order). Rows
// of 32 or more entries on average take spmv_wave_kernel: one wave per RW consecutive
// rows, 64 lanes per row, with the RW rows' loads issued together so that each wave
// keeps RW independent col/val -> x load chains in flight. Each entry's x gather is a
// separate L2 request (x stays in L2), and that request rate, not HBM bandwidth, is
// what bounds SpMV at C5's sparsity.
#include "common.h"

namespace gn {
namespace {

typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kBlock = 256;  // 4 waves

__device__ __forceinline__ void row_bounds(const int32_t *rowptr, long row, long nnz, int &s, int &e, int *flags,
                                           bool leader) {
  s = rowptr[row];
  e = rowptr[row + 1];
  if (s < 0 || e < s || (long)e > nnz) {
    if (leader && flags) flags[0] = 1;
    s = e = 0;
  }
}

template <int LPR>
__global__ void __launch_bounds__(kBlock) spmm_vec4_kernel(long M, long N, long K, long nnz,
                                                           const int32_t *__restrict__ rowptr,
                                                           const int32_t *__restrict__ col,
                                                           const float *__restrict__ val,
                                                           const float *__restrict__ D, long ldd,
                                                           float *__restrict__ C, long ldc, int *flags) {
  constexpr int RPW = 64 / LPR;  // rows per wave
  const int lane = threadIdx.x & 63;
  const int li = lane % LPR;
  long row = ((long)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6)) * RPW + lane / LPR;
  if (LPR == 64) row = __builtin_amdgcn_readfirstlane((int)row);  // one row per wave: make it uniform
  if (row >= M) return;
  int s, e;
  row_bounds(rowptr, row, nnz, s, e, flags, li == 0);
  for (long c0 = 4L * li; c0 < N; c0 += 4L * LPR) {
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
    int k = s;
    for (; k + 4 <= e; k += 4) {
      int cc[4];
      float vv[4];
      float4_t dd[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        cc[u] = col[k + u];
        vv[u] = val[k + u];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool ok = (unsigned)cc[u] < (unsigned long)K;
        dd[u] = ok ? *reinterpret_cast<const float4_t *>(D + (long)cc[u] * ldd + c0) : float4_t{0.f, 0.f, 0.f, 0.f};
        if (!ok) {
          vv[u] = 0.f;
          if (flags) flags[1] = 1;
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if ((unsigned)cc[u] < (unsigned long)K) {
          acc[0] = __builtin_fmaf(vv[u], dd[u][0], acc[0]);
          acc[1] = __builtin_fmaf(vv[u], dd[u][1], acc[1]);
          acc[2] = __builtin_fmaf(vv[u], dd[u][2], acc[2]);
          acc[3] = __builtin_fmaf(vv[u], dd[u][3], acc[3]);
        }
      }
    }
    for (; k < e; ++k) {
      const int c = col[k];
      if ((unsigned)c < (unsigned long)K) {
        const float v = val[k];
        const float4_t d = *reinterpret_cast<const float4_t *>(D + (long)c * ldd + c0);
        acc[0] = __builtin_fmaf(v, d[0], acc[0]);
        acc[1] = __builtin_fmaf(v, d[1], acc[1]);
        acc[2] = __builtin_fmaf(v, d[2], acc[2]);
        acc[3] = __builtin_fmaf(v, d[3], acc[3]);
      } else if (flags) {
        flags[1] = 1;
      }
    }
    *reinterpret_cast<float4_t *>(C + row * ldc + c0) = acc;
  }
}

// Element-wise variant for N or pitches that are not multiples of 4 floats.
template <int LPR>
__global__ void __launch_bounds__(kBlock) spmm_scalar_kernel(long M, long N, long K, long nnz,
                                                             const int32_t *__restrict__ rowptr,
                                                             const int32_t *__restrict__ col,
                                                             const float *__restrict__ val,
                                                             const float *__restrict__ D, long ldd,
                                                             float *__restrict__ C, long ldc, int *flags) {
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int li = lane % LPR;
  const long row = ((long)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6)) * RPW + lane / LPR;
  if (row >= M) return;
  int s, e;
  row_bounds(rowptr, row, nnz, s, e, flags, li == 0);
  for (long c0 = li; c0 < N; c0 += LPR) {
    float acc = 0.f;
    for (int k = s; k < e; ++k) {
      const int c = col[k];
      if ((unsigned)c < (unsigned long)K) acc = __builtin_fmaf(val[k], D[(long)c * ldd + c0], acc);
      else if (flags) flags[1] = 1;
    }
    C[row * ldc + c0] = acc;
  }
}

// Column-banded SpMM for N >= 32 (16-byte aligned D and C rows). The output columns are
// cut into bands of kBandCols = 32 floats, one 128-byte L2 line of each D row; 8 lanes
// own a (row, band) pair, 4 columns each, so a wave covers 8 rows of one band and each
// gather instruction touches 8 whole lines. Workgroups run band-major (all row blocks of
// band 0, then band 1, ...), so the workgroups resident at any time gather from one or
// two bands of D: an 8 MiB working set per band at N = 256 instead of all of D. The
// entries of a row are consumed in CSR order in batches of kBandUnroll, whose index
// loads and gathers are all issued before the first fma; a row's last entries go one
// at a time. Every output is the same fma chain as in spmm_vec4_kernel.
constexpr int kBandCols = 32;
constexpr int kBandLanes = kBandCols / 4;
constexpr int kBandRowsPerBlock = (kBlock / 64) * (64 / kBandLanes);
constexpr int kBandUnroll = 16;
constexpr long kSplitMinNnz = 1L << 16;  // below this, one launch of spmm_band_kernel

__global__ void __launch_bounds__(kBlock) spmm_band_kernel(long M, long N, long K, long nnz, long row_blocks,
                                                           const int32_t *__restrict__ rowptr,
                                                           const int32_t *__restrict__ col,
                                                           const float *__restrict__ val,
                                                           const float *__restrict__ D, long ldd,
                                                           float *__restrict__ C, long ldc, int *flags) {
  const int lane = threadIdx.x & 63;
  const int li = lane % kBandLanes;
  const long band = blockIdx.x / row_blocks;
  const long row = (blockIdx.x % row_blocks) * kBandRowsPerBlock + (threadIdx.x >> 6) * (64 / kBandLanes) +
                   lane / kBandLanes;
  const long c0 = band * kBandCols + 4 * li;
  // No cross-lane operations follow, so lanes past the last row or column leave here.
  if (row >= M || c0 >= N) return;
  int s, e;
  row_bounds(rowptr, row, nnz, s, e, flags, li == 0);
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
  bool bad_col = false;
  int k = s;
  for (; k + kBandUnroll <= e; k += kBandUnroll) {
    int cc[kBandUnroll];
    float vv[kBandUnroll];
    float4_t dd[kBandUnroll];
#pragma unroll
    for (int u = 0; u < kBandUnroll; ++u) {
      cc[u] = col[k + u];
      vv[u] = val[k + u];
    }
    unsigned ok = 0;  // bit u: entry k+u has a column inside D
#pragma unroll
    for (int u = 0; u < kBandUnroll; ++u) {
      if ((unsigned)cc[u] < (unsigned long)K) {
        dd[u] = *reinterpret_cast<const float4_t *>(D + (long)cc[u] * ldd + c0);
        ok |= 1u << u;
      }
    }
    bad_col |= ok != (1u << kBandUnroll) - 1;
#pragma unroll
    for (int u = 0; u < kBandUnroll; ++u) {
      if (ok & (1u << u)) {
        acc[0] = __builtin_fmaf(vv[u], dd[u][0], acc[0]);
        acc[1] = __builtin_fmaf(vv[u], dd[u][1], acc[1]);
        acc[2] = __builtin_fmaf(vv[u], dd[u][2], acc[2]);
        acc[3] = __builtin_fmaf(vv[u], dd[u][3], acc[3]);
      }
    }
  }
  for (; k < e; ++k) {
    const int c = col[k];
    if ((unsigned)c < (unsigned long)K) {
      const float v = val[k];
      const float4_t d = *reinterpret_cast<const float4_t *>(D + (long)c * ldd + c0);
      acc[0] = __builtin_fmaf(v, d[0], acc[0]);
      acc[1] = __builtin_fmaf(v, d[1], acc[1]);
      acc[2] = __builtin_fmaf(v, d[2], acc[2]);
      acc[3] = __builtin_fmaf(v, d[3], acc[3]);
    } else {
      bad_col = true;
    }
  }
  if (bad_col && flags) flags[1] = 1;
  *reinterpret_cast<float4_t *>(C + row * ldc + c0) = acc;
}

// The band kernel in two launches over each row's entries: launch 0 sums entries s .. p-1
// into C, launch 1 loads that partial and adds entries p .. e-1, so each output still takes
// one fma per entry in CSR order (the partial is stored exactly) and the result is
// bit-identical to one launch for any split point p. CUT: p is the row's first entry whose
// column reaches kcut (K / 2), found by launch 0 and passed to launch 1 through split[row]
// (written by the row's band-0 lanes); otherwise p is the midpoint of the row's entries. With
// sorted columns either split keeps each launch's gathers in about half of D's rows; the
// column cut does so exactly. Batches of 16 entries may read indices and values past the
// row's end (never past nnz) and mask them, so no row ends in a one-entry-at-a-time tail;
// only the last entries of the arrays take it.
template <bool SECOND, bool CUT>
__global__ void __launch_bounds__(kBlock) spmm_band_half_kernel(long M, long N, long K, long nnz, long row_blocks,
                                                                const int32_t *__restrict__ rowptr,
                                                                const int32_t *__restrict__ col,
                                                                const float *__restrict__ val,
                                                                const float *__restrict__ D, long ldd,
                                                                float *__restrict__ C, long ldc, int *flags, int kcut,
                                                                int *__restrict__ split) {
  const int lane = threadIdx.x & 63;
  const int li = lane % kBandLanes;
  const long band = blockIdx.x / row_blocks;
  const long row = (blockIdx.x % row_blocks) * kBandRowsPerBlock + (threadIdx.x >> 6) * (64 / kBandLanes) +
                   lane / kBandLanes;
  const long c0 = band * kBandCols + 4 * li;
  if (row >= M || c0 >= N) return;
  int s, e;
  row_bounds(rowptr, row, nnz, s, e, flags, li == 0 && !SECOND);
  int lo, hi;
  if constexpr (CUT) {
    lo = SECOND ? split[row] : s;  // launch 0 wrote a position in [s, e]
    hi = e;
  } else {
    const int m = s + ((e - s) >> 1);
    lo = SECOND ? m : s;
    hi = SECOND ? e : m;
  }
  constexpr bool STOP = CUT && !SECOND;  // launch 0 of the column cut ends at the first column >= kcut
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
  if (SECOND) acc = *reinterpret_cast<const float4_t *>(C + row * ldc + c0);
  bool bad_col = false, cut = false;
  int k = lo;
  while (k < hi && k + kBandUnroll <= nnz) {
    int cc[kBandUnroll];
    float vv[kBandUnroll];
    float4_t dd[kBandUnroll];
#pragma unroll
    for (int u = 0; u < kBandUnroll; ++u) {
      cc[u] = col[k + u];
      vv[u] = val[k + u];
    }
    int f = hi - k < kBandUnroll ? hi - k : kBandUnroll;  // entries of this range in the batch
    if constexpr (STOP) {
      int g = kBandUnroll;
#pragma unroll
      for (int u = kBandUnroll - 1; u >= 0; --u)
        if (cc[u] >= kcut) g = u;
      if (g < f) f = g, cut = true;
    }
    unsigned ok = 0;
#pragma unroll
    for (int u = 0; u < kBandUnroll; ++u) {
      if (u < f && (unsigned)cc[u] < (unsigned long)K) {
        dd[u] = *reinterpret_cast<const float4_t *>(D + (long)cc[u] * ldd + c0);
        ok |= 1u << u;
      }
    }
    bad_col |= ok != (f == kBandUnroll ? (1u << kBandUnroll) - 1 : (1u << f) - 1);
#pragma unroll
    for (int u = 0; u < kBandUnroll; ++u) {
      if (ok & (1u << u)) {
        acc[0] = __builtin_fmaf(vv[u], dd[u][0], acc[0]);
        acc[1] = __builtin_fmaf(vv[u], dd[u][1], acc[1]);
        acc[2] = __builtin_fmaf(vv[u], dd[u][2], acc[2]);
        acc[3] = __builtin_fmaf(vv[u], dd[u][3], acc[3]);
      }
    }
    k += f;
    if (cut) break;
  }
  for (; !cut && k < hi; ++k) {  // within 16 entries of the end of the arrays
    const int c = col[k];
    if (STOP && c >= kcut) break;
    if ((unsigned)c < (unsigned long)K) {
      const float v = val[k];
      const float4_t d = *reinterpret_cast<const float4_t *>(D + (long)c * ldd + c0);
      acc[0] = __builtin_fmaf(v, d[0], acc[0]);
      acc[1] = __builtin_fmaf(v, d[1], acc[1]);
      acc[2] = __builtin_fmaf(v, d[2], acc[2]);
      acc[3] = __builtin_fmaf(v, d[3], acc[3]);
    } else {
      bad_col = true;
    }
  }
  if (STOP && band == 0 && li == 0) split[row] = k;
  if (bad_col && flags) flags[1] = 1;
  *reinterpret_cast<float4_t *>(C + row * ldc + c0) = acc;
}

template <int LPR>
__global__ void __launch_bounds__(kBlock) spmv_kernel(long M, long K, long nnz, const int32_t *__restrict__ rowptr,
                                                      const int32_t *__restrict__ col,
                                                      const float *__restrict__ val, const float *__restrict__ x,
                                                      float *__restrict__ y, int *flags) {
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int li = lane % LPR;
  const long row = ((long)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6)) * RPW + lane / LPR;
  // Lanes past M still take part in the shuffles below (with an empty row).
  int s = 0, e = 0;
  if (row < M) row_bounds(rowptr, row, nnz, s, e, flags, li == 0);
  float acc = 0.f;
  for (int k = s + li; k < e; k += LPR) {
    const int c = col[k];
    if ((unsigned)c < (unsigned long)K) acc = __builtin_fmaf(val[k], x[c], acc);
    else if (flags) flags[1] = 1;
  }
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (row < M && li == 0) y[row] = acc;
}

int next_pow2_lanes(long n) {
  int l = 1;
  while (l < 64 && l < n) l <<= 1;
  return l;
}

}  // namespace

int launch_spmm(long M, long N, long K, long nnz, const int32_t *rowptr, const int32_t *col, const float *val,
                const float *D, long ldd, float *C, long ldc, int *flags, hipStream_t s, CError *err) {
  if (M < 0 || N < 0 || K < 0 || nnz < 0) return set_error(err, -1, "spmm: negative size");
  if (M == 0 || N == 0) return 0;
  if (!rowptr || !C || (nnz > 0 && (!col || !val)) || (K > 0 && !D)) return set_error(err, -1, "spmm: NULL pointer");
  if (ldd < N || ldc < N) return set_error(err, -1, "spmm: leading dimension smaller than N");
  if (nnz > 0x7FFFFFFFL || M > 0x7FFFFFF0L) return set_error(err, -1, "spmm: exceeds int32 CSR indexing");
  const bool vec = N % 4 == 0 && ldd % 4 == 0 && ldc % 4 == 0 && (uintptr_t)D % 16 == 0 && (uintptr_t)C % 16 == 0;
  if (vec && N >= kBandCols) {
    const long row_blocks = (M + kBandRowsPerBlock - 1) / kBandRowsPerBlock;
    const long bands = (N + kBandCols - 1) / kBandCols;
    if (row_blocks > 0x7FFFFFFFL / bands) return set_error(err, -1, "spmm: too many rows");
    const dim3 g((unsigned)(row_blocks * bands)), b(kBlock);
    if (nnz >= kSplitMinNnz) {
      // Two launches. With the rows split at their entries' midpoint, C5 (65536^2, 4.3 M
      // entries, N = 256): 463 -> 383 us against one launch; 16 entries per row 218 -> 144 us;
      // N = 32 65 -> 54 us; K = 16384 313 -> 280 us; K = 131072 580 -> 563 us; bit-identical to
      // one launch in every case. The column cut needs the M split positions between the
      // launches, in the stream's scratch, so graph capture (where that may allocate) keeps
      // the midpoint.
      hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
      std::unique_lock<std::mutex> lk;
      int *split = nullptr;
      if (hipStreamIsCapturing(s, &cap) == hipSuccess && cap == hipStreamCaptureStatusNone) {
        split = static_cast<int *>(stream_scratch(s, (size_t)M * sizeof(int), lk, err));
        if (!split) return -3;
      }
      const int kcut = (int)std::min<long>(K / 2, 0x7FFFFFFFL);  // columns are int32
      if (split) {
        hipLaunchKernelGGL((spmm_band_half_kernel<false, true>), g, b, 0, s, M, N, K, nnz, row_blocks, rowptr, col, val,
                           D, ldd, C, ldc, flags, kcut, split);
        hipLaunchKernelGGL((spmm_band_half_kernel<true, true>), g, b, 0, s, M, N, K, nnz, row_blocks, rowptr, col, val,
                           D, ldd, C, ldc, flags, kcut, split);
      } else {
        hipLaunchKernelGGL((spmm_band_half_kernel<false, false>), g, b, 0, s, M, N, K, nnz, row_blocks, rowptr, col,
                           val, D, ldd, C, ldc, flags, kcut, split);
        hipLaunchKernelGGL((spmm_band_half_kernel<true, false>), g, b, 0, s, M, N, K, nnz, row_blocks, rowptr, col, val,
                           D, ldd, C, ldc, flags, kcut, split);
      }
    } else {
      hipLaunchKernelGGL(spmm_band_kernel, g, b, 0, s, M, N, K, nnz, row_blocks, rowptr, col, val, D, ldd, C, ldc,
                         flags);
    }
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : hip_error(err, -6, "spmm launch", e);
  }
  const int lpr = next_pow2_lanes(vec ? (N + 3) / 4 : N);
  const long rows_per_block = (kBlock / 64) * (64 / lpr);
  const long blocks = (M + rows_per_block - 1) / rows_per_block;
  if (blocks > 0x7FFFFFFFL) return set_error(err, -1, "spmm: too many rows");
  dim3 g((unsigned)blocks), b(kBlock);
#define GN_SPMM_CASE(L)                                                                                         \
  case L:                                                                                                       \
    if (vec) hipLaunchKernelGGL(spmm_vec4_kernel<L>, g, b, 0, s, M, N, K, nnz, rowptr, col, val, D, ldd, C, ldc, \
                                flags);                                                                         \
    else hipLaunchKernelGGL(spmm_scalar_kernel<L>, g, b, 0, s, M, N, K, nnz, rowptr, col, val, D, ldd, C, ldc,  \
                            flags);                                                                             \
    break;
  switch (lpr) {
    GN_SPMM_CASE(1)
    GN_SPMM_CASE(2)
    GN_SPMM_CASE(4)
    GN_SPMM_CASE(8)
    GN_SPMM_CASE(16)
    GN_SPMM_CASE(32)
    GN_SPMM_CASE(64)
  }
#undef GN_SPMM_CASE
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : hip_error(err, -6, "spmm launch", e);
}

namespace {

// Lane l of a row sums entries s+l, s+l+64, ... in order; the shuffle tree then gives
// the same result, bit for bit, as spmv_kernel<64>.
template <int RW>
__global__ void __launch_bounds__(kBlock) spmv_wave_kernel(long M, long K, long nnz, const int32_t *__restrict__ rowptr,
                                                           const int32_t *__restrict__ col,
                                                           const float *__restrict__ val, const float *__restrict__ x,
                                                           float *__restrict__ y, int *flags) {
  const int lane = threadIdx.x & 63;
  const long r0 = (long)__builtin_amdgcn_readfirstlane((int)(blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6))) * RW;
  if (r0 >= M) return;  // the whole wave
  int s[RW], e[RW];
  int maxlen = 0;
#pragma unroll
  for (int u = 0; u < RW; ++u) {
    s[u] = e[u] = 0;
    if (r0 + u < M) row_bounds(rowptr, r0 + u, nnz, s[u], e[u], flags, lane == 0);
    maxlen = max(maxlen, e[u] - s[u]);
  }
  float acc[RW];
#pragma unroll
  for (int u = 0; u < RW; ++u) acc[u] = 0.f;
  for (int base = 0; base < maxlen; base += 64) {
    int cc[RW];
    float vv[RW], xx[RW];
#pragma unroll
    for (int u = 0; u < RW; ++u) {
      const int k = s[u] + base + lane;
      cc[u] = -1;
      vv[u] = 0.f;
      if (k < e[u]) {
        cc[u] = col[k];
        vv[u] = val[k];
      }
    }
#pragma unroll
    for (int u = 0; u < RW; ++u) {
      const bool ok = (unsigned)cc[u] < (unsigned long)K;
      xx[u] = ok ? x[cc[u]] : 0.f;
      if (!ok && cc[u] != -1 && flags) flags[1] = 1;
    }
#pragma unroll
    for (int u = 0; u < RW; ++u)
      if ((unsigned)cc[u] < (unsigned long)K) acc[u] = __builtin_fmaf(vv[u], xx[u], acc[u]);
  }
#pragma unroll
  for (int u = 0; u < RW; ++u) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc[u] += __shfl_xor(acc[u], off, 64);
    if (lane == 0 && r0 + u < M) y[r0 + u] = acc[u];
  }
}

}  // namespace

int launch_spmv(long M, long K, long nnz, const int32_t *rowptr, const int32_t *col, const float *val,
                const float *x, float *y, int *flags, hipStream_t s, CError *err) {
  if (M < 0 || K < 0 || nnz < 0) return set_error(err, -1, "spmv: negative size");
  if (M == 0) return 0;
  if (!rowptr || !y || (nnz > 0 && (!col || !val)) || (K > 0 && !x)) return set_error(err, -1, "spmv: NULL pointer");
  if (nnz > 0x7FFFFFFFL || M > 0x7FFFFFF0L) return set_error(err, -1, "spmv: exceeds int32 CSR indexing");
  // Lanes per row from the mean row length (clamped to 4..64).
  const long mean = nnz / M;
  int lpr = 4;
  while (lpr < 64 && lpr * 2 <= mean / 2) lpr <<= 1;
  if (mean >= 32) {
    constexpr int RW = 2;
    const long blocks = (M + (kBlock / 64) * RW - 1) / ((kBlock / 64) * RW);
    if (blocks > 0x7FFFFFFFL / (kBlock / 64)) return set_error(err, -1, "spmv: too many rows");
    hipLaunchKernelGGL(spmv_wave_kernel<RW>, dim3((unsigned)blocks), dim3(kBlock), 0, s, M, K, nnz, rowptr, col, val, x,
                       y, flags);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : hip_error(err, -6, "spmv launch", e);
  }
  const long rows_per_block = (kBlock / 64) * (64 / lpr);
  const long blocks = (M + rows_per_block - 1) / rows_per_block;
  if (blocks > 0x7FFFFFFFL) return set_error(err, -1, "spmv: too many rows");
  dim3 g((unsigned)blocks), b(kBlock);
  switch (lpr) {
    case 4: hipLaunchKernelGGL(spmv_kernel<4>, g, b, 0, s, M, K, nnz, rowptr, col, val, x, y, flags); break;
    case 8: hipLaunchKernelGGL(spmv_kernel<8>, g, b, 0, s, M, K, nnz, rowptr, col, val, x, y, flags); break;
    case 16: hipLaunchKernelGGL(spmv_kernel<16>, g, b, 0, s, M, K, nnz, rowptr, col, val, x, y, flags); break;
    case 32: hipLaunchKernelGGL(spmv_kernel<32>, g, b, 0, s, M, K, nnz, rowptr, col, val, x, y, flags); break;
    default: hipLaunchKernelGGL(spmv_kernel<64>, g, b, 0, s, M, K, nnz, rowptr, col, val, x, y, flags); break;
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : hip_error(err, -6, "spmv launch", e);
}

}  // namespace gn
