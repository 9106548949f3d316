// spmv_grouped.hip — CSR SpMV over a one-time "grouped" layout of the sparsity structure.
//
// The flat SpMV kernels (sparse.hip) gather x[col] entry by entry in CSR order: within a
// row the columns are spread over all of x, so each lane of a gather instruction touches
// its own 128-byte line and every stored entry costs one L2 request; that request rate, not
// HBM, bounds them (C5: 0.99 requests per entry). This layout regroups the gathers:
//
//  * the rows are cut into blocks of consecutive rows, about nnz / (blocks) entries each,
//    with the number of blocks a multiple of the CU count (one round of workgroups), every
//    block at most kCap entries; structures with a row longer than kMaxRow entries get no
//    layout (a sequential sum over such a row would dominate the launch) and keep the flat
//    kernel;
//  * inside a block the entries are ordered by the 128-byte line of x their column falls in
//    (a counting sort on col >> shift, done once on the GPU). For K <= 65536 each grouped
//    entry is one 32-bit word: column (bits 0-15), its position in the block's CSR order
//    (bits 16-30) and an out-of-range flag (bit 31); wider x keeps the column (int32) and
//    the position (uint16) in two arrays.
//
// spmv_grouped_kernel (one workgroup of 1024 threads per block) issues each thread's whole
// share of the block's layout and value loads at once, then all its x gathers (the 64
// lanes of an instruction share a few lines), then writes each gathered value into LDS at
// its CSR position next to the block's values; after a barrier every row is summed
// sequentially in CSR order with one fma per entry: bit-identical to the reference loop
// (metal_bridge_sparse.m:327-339) restated with fmaf. Columns outside [0, K) contribute
// nothing and raise flags[1]. Every LDS and layout index is bounded by the layout's own
// block offsets, and row bounds read from the row pointers are clamped to the block, so a
// row-pointer array that no longer matches the layout gives wrong sums, never an access
// outside the arrays.
#include <algorithm>
#include <vector>

#include "common.h"

namespace gn {
namespace {

constexpr int kThreads = 1024;   // 16 waves: many gathers in flight per CU
constexpr int kCap = 20476;      // entries per block: x values, values and 4 spare floats in 160 KiB of LDS
constexpr int kMaxRow = 4096;    // longest row the layout takes
constexpr int kMaxBins = 4096;   // counting-sort bins (16 KiB of LDS)
constexpr uint32_t kBadBit = 0x80000000u;
typedef float float4_t __attribute__((ext_vector_type(4)));

// Exclusive prefix sum of n <= kMaxBins ints in LDS, by the whole block (kThreads threads).
__device__ void block_exclusive_scan(int *a, int n, int *wave_tot) {
  constexpr int kPer = kMaxBins / kThreads;  // bins per thread
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  int v[kPer];
  int sum = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int idx = t * kPer + i;
    v[i] = idx < n ? a[idx] : 0;
    sum += v[i];
  }
  // inclusive scan of the per-thread sums across the wave
  int inc = sum;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(inc, off, 64);
    if (lane >= off) inc += o;
  }
  if (lane == 63) wave_tot[w] = inc;
  __syncthreads();
  if (t == 0) {
    int run = 0;
    for (int i = 0; i < kThreads / 64; ++i) {
      const int c = wave_tot[i];
      wave_tot[i] = run;
      run += c;
    }
  }
  __syncthreads();
  int base = wave_tot[w] + inc - sum;  // exclusive prefix of this thread's first bin
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int idx = t * kPer + i;
    if (idx < n) a[idx] = base;
    base += v[i];
  }
  __syncthreads();
}

// One workgroup per block: the block's entries grouped by col >> shift (out-of-range
// columns in bin 0). blk_ent holds the blocks' entry offsets (n <= kCap each).
template <bool PACKED>
__global__ void __launch_bounds__(kThreads) spmv_group_sort_kernel(const int32_t *__restrict__ blk_ent,
                                                                   const int32_t *__restrict__ col, long K, int shift,
                                                                   int nbins, uint32_t *__restrict__ word,
                                                                   int32_t *__restrict__ scol,
                                                                   uint16_t *__restrict__ spos) {
  __shared__ int hist[kMaxBins];
  __shared__ int wave_tot[kThreads / 64];
  const int e0 = blk_ent[blockIdx.x], n = blk_ent[blockIdx.x + 1] - e0;
  for (int i = threadIdx.x; i < nbins; i += kThreads) hist[i] = 0;
  __syncthreads();
  for (int j = threadIdx.x; j < n; j += kThreads) {
    const int c = col[e0 + j];
    const int key = (unsigned)c < (unsigned long)K ? (c >> shift) : 0;
    atomicAdd(&hist[key], 1);
  }
  __syncthreads();
  block_exclusive_scan(hist, nbins, wave_tot);
  // Within a bin the order is whatever the atomics give: it only decides which lane gathers
  // which value; every value lands at its CSR position, so the result does not depend on it.
  for (int j = threadIdx.x; j < n; j += kThreads) {
    const int c = col[e0 + j];
    const bool ok = (unsigned)c < (unsigned long)K;
    const int p = atomicAdd(&hist[ok ? (c >> shift) : 0], 1);
    if (PACKED) {
      word[e0 + p] = (ok ? 0u : kBadBit) | ((uint32_t)j << 16) | (ok ? (uint32_t)c : 0u);
    } else {
      scol[e0 + p] = c;
      spos[e0 + p] = (uint16_t)j;
    }
  }
}

// y[r] for the rows of one block; R * kThreads >= the block's entries. LDS: xs[cap4] (x
// values at CSR positions), vs[cap4] (values; cap4 = cap rounded up to 4, so both arrays
// are 16-byte aligned), and spare floats that lanes past the block write to (so the stores
// need no branch the gathers could be sunk into).
template <int R, bool PACKED>
__global__ void __launch_bounds__(kThreads) spmv_grouped_kernel(long K, const int32_t *__restrict__ rowptr,
                                                                const int32_t *__restrict__ blk_row,
                                                                const int32_t *__restrict__ blk_ent,
                                                                const uint32_t *__restrict__ word,
                                                                const int32_t *__restrict__ scol,
                                                                const uint16_t *__restrict__ spos,
                                                                const float *__restrict__ val,
                                                                const float *__restrict__ x, float *__restrict__ y,
                                                                int cap, int *flags) {
  extern __shared__ float lds[];
  const int cap4 = (cap + 3) & ~3;
  const int spare = 2 * cap4;  // lds[spare]
  const int t = threadIdx.x;
  const int r0 = blk_row[blockIdx.x], r1 = blk_row[blockIdx.x + 1];
  const int e0 = blk_ent[blockIdx.x];
  const int n = min(blk_ent[blockIdx.x + 1] - e0, min(cap, R * kThreads));  // equal when built
  bool bad = false;
  if (n > 0) {
    int cc[R], pp[R];
    float vv[R], xv[R];
    // Three phases kept apart by scheduling barriers: every layout and value load of the
    // thread (indices past the block repeat its last entry), then every x gather, then the
    // LDS stores; each thread waits for memory twice, not once per entry.
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int q = e0 + min(t + i * kThreads, n - 1);
      if (PACKED) {
        const uint32_t w = word[q];
        cc[i] = (w & kBadBit) ? -1 : (int)(w & 0xFFFFu);
        pp[i] = (int)((w >> 16) & 0x7FFFu);
      } else {
        cc[i] = scol[q];
        pp[i] = spos[q];
      }
    }
#pragma unroll
    for (int i = 0; i < R; ++i) vv[i] = val[e0 + min(t + i * kThreads, n - 1)];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const bool ok = (unsigned)cc[i] < (unsigned long)K;
      bad |= !ok;
      const float g = x[ok ? cc[i] : 0];
      xv[i] = ok ? g : 0.0f;  // an out-of-range column contributes fma(v, 0, sum)
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int j = t + i * kThreads;
      lds[j < n ? cap4 + j : spare] = vv[i];
    }
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int j = t + i * kThreads;
      // pp is a permutation of [0, n) when built; anything else goes to the spare slot
      lds[(j < n && (unsigned)pp[i] < (unsigned)n) ? pp[i] : spare] = xv[i];
    }
  }
  __syncthreads();
  for (int r = r0 + t; r < r1; r += kThreads) {
    int s = rowptr[r] - e0, e = rowptr[r + 1] - e0;
    s = max(0, min(s, n));
    e = max(s, min(e, n));
    // One fma per entry in CSR order, the entries read as 16-byte groups of four (entry
    // 4g..4g+3): the lanes' rows start at unrelated banks, and the LDS then moves four
    // entries per conflict cycle instead of one or two (C5's row sums 5,700 -> 3,400 cycles
    // per wave). Entries of the first and last group outside [s, e) leave a unchanged (a
    // select, so a row whose partial sum is -0 keeps it); those of a group past the block
    // lie inside the arrays' cap4 extent and are not used.
    float a = 0.0f;
    if (s < e) {
      const float4_t *v4 = reinterpret_cast<const float4_t *>(lds + cap4);
      const float4_t *x4 = reinterpret_cast<const float4_t *>(lds);
      int g = s >> 2;
      const int g_end = (e + 3) >> 2;
      {
        const float4_t vv = v4[g], xx = x4[g];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int k = 4 * g + u;
          const float f = __builtin_fmaf(vv[u], xx[u], a);
          a = (k >= s && k < e) ? f : a;
        }
        ++g;
      }
      for (; g + 2 < g_end; g += 2) {  // two whole groups
        const float4_t va = v4[g], xa = x4[g], vb = v4[g + 1], xb = x4[g + 1];
#pragma unroll
        for (int u = 0; u < 4; ++u) a = __builtin_fmaf(va[u], xa[u], a);
#pragma unroll
        for (int u = 0; u < 4; ++u) a = __builtin_fmaf(vb[u], xb[u], a);
      }
      for (; g < g_end; ++g) {  // at most two more, the last one possibly partial
        const float4_t vv = v4[g], xx = x4[g];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float f = __builtin_fmaf(vv[u], xx[u], a);
          a = (4 * g + u < e) ? f : a;
        }
      }
    }
    y[r] = a;
  }
  if (bad && flags) flags[1] = 1;
}

template <bool PACKED>
hipError_t launch_grouped(const SpmvLayout &l, const int32_t *rowptr, const float *val, const float *x, float *y,
                          int *flags, hipStream_t s) {
  const size_t lds = sizeof(float) * (2 * (((size_t)l.cap + 3) & ~(size_t)3) + 4);
  const int need = (l.cap + kThreads - 1) / kThreads;
  const int32_t *blk_ent = l.blk + (l.nblocks + 1);
#define GN_GROUPED_CASE(RR)                                                                                   \
  if (need <= RR) {                                                                                           \
    hipLaunchKernelGGL((spmv_grouped_kernel<RR, PACKED>), dim3((unsigned)l.nblocks), dim3(kThreads), lds, s, \
                       l.K, rowptr, l.blk, blk_ent, l.word, l.scol, l.spos, val, x, y, l.cap, flags);          \
    return hipGetLastError();                                                                                 \
  }
  GN_GROUPED_CASE(1)
  GN_GROUPED_CASE(2)
  GN_GROUPED_CASE(4)
  GN_GROUPED_CASE(8)
  GN_GROUPED_CASE(12)
  GN_GROUPED_CASE(16)
  GN_GROUPED_CASE(20)
#undef GN_GROUPED_CASE
  return hipErrorInvalidValue;  // cap <= kCap = 20 * kThreads when built
}

}  // namespace

bool spmv_grouped_supported(long M, long K, long nnz) {
  return M > 0 && K > 0 && nnz > 0 && nnz <= 0x7FFFFFFFL && M < 0x7FFFFFF0L;
}

int build_spmv_layout(long M, long K, long nnz, const int32_t *h_rowptr, const int32_t *d_col, int num_cus,
                      hipStream_t s, SpmvLayout *out, CError *err) {
  *out = SpmvLayout{};
  if (!spmv_grouped_supported(M, K, nnz)) return 1;
  long maxrow = 0;
  for (long r = 0; r < M; ++r) maxrow = std::max<long>(maxrow, (long)h_rowptr[r + 1] - h_rowptr[r]);
  if (maxrow > kMaxRow) return 1;
  // Row blocks: at most a multiple of the CU count of them, each at most kCap entries
  // (every row fits: kMaxRow <= kCap / 2).
  const long cus = std::max(1, num_cus);
  long nb = cus;
  while ((nnz + nb - 1) / nb + maxrow > kCap) nb += cus;
  const long target = (nnz + nb - 1) / nb + maxrow;
  std::vector<int32_t> rows, ents;
  rows.reserve((size_t)nb + 2);
  ents.reserve((size_t)nb + 2);
  rows.push_back(0);
  ents.push_back(h_rowptr[0]);
  long acc = 0, biggest = 0;
  for (long r = 0; r < M; ++r) {
    const long len = (long)h_rowptr[r + 1] - h_rowptr[r];
    if (acc > 0 && acc + len > target) {
      rows.push_back((int32_t)r);
      ents.push_back(h_rowptr[r]);
      biggest = std::max(biggest, acc);
      acc = 0;
    }
    acc += len;
  }
  rows.push_back((int32_t)M);
  ents.push_back(h_rowptr[M]);
  biggest = std::max(biggest, acc);
  const int nblocks = (int)rows.size() - 1;
  // Sort key: the 128-byte line of x (32 floats), coarser when that needs more bins.
  int shift = 5;
  while (((K - 1) >> shift) + 1 > kMaxBins) ++shift;
  const int nbins = (int)(((K - 1) >> shift) + 1);
  const bool packed = K <= 65536;
  out->M = M;
  out->K = K;
  out->nnz = nnz;
  out->nblocks = nblocks;
  out->cap = (int)std::max<long>(biggest, 1);
  std::vector<int32_t> blk(rows);
  blk.insert(blk.end(), ents.begin(), ents.end());
  out->blk = static_cast<int32_t *>(dev_alloc(sizeof(int32_t) * blk.size(), err));
  bool ok = out->blk != nullptr;
  if (ok && packed) {
    out->word = static_cast<uint32_t *>(dev_alloc(sizeof(uint32_t) * (size_t)nnz, err));
    ok = out->word != nullptr;
  } else if (ok) {
    out->scol = static_cast<int32_t *>(dev_alloc(sizeof(int32_t) * (size_t)nnz, err));
    out->spos = static_cast<uint16_t *>(dev_alloc(sizeof(uint16_t) * (size_t)nnz, err));
    ok = out->scol && out->spos;
  }
  if (!ok) {
    free_spmv_layout(out, s);
    return -3;
  }
  if (int rc = upload(out->blk, blk.data(), sizeof(int32_t) * blk.size(), s, err)) {
    free_spmv_layout(out, s);
    return rc;
  }
  const int32_t *d_ent = out->blk + (nblocks + 1);
  if (packed)
    hipLaunchKernelGGL(spmv_group_sort_kernel<true>, dim3((unsigned)nblocks), dim3(kThreads), 0, s, d_ent, d_col, K,
                       shift, nbins, out->word, out->scol, out->spos);
  else
    hipLaunchKernelGGL(spmv_group_sort_kernel<false>, dim3((unsigned)nblocks), dim3(kThreads), 0, s, d_ent, d_col, K,
                       shift, nbins, out->word, out->scol, out->spos);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    free_spmv_layout(out, s);
    return hip_error(err, -6, "spmv layout launch", e);
  }
  return 0;
}

void free_spmv_layout(SpmvLayout *l, hipStream_t s) {
  dev_free_on(l->blk, s);
  dev_free_on(l->word, s);
  dev_free_on(l->scol, s);
  dev_free_on(l->spos, s);
  *l = SpmvLayout{};
}

int launch_spmv_grouped(const SpmvLayout &l, const int32_t *d_rowptr, const float *val, const float *x, float *y,
                        int *flags, hipStream_t s, CError *err) {
  if (!l.blk) return set_error(err, -1, "spmv: no layout");
  const hipError_t e = l.word ? launch_grouped<true>(l, d_rowptr, val, x, y, flags, s)
                              : launch_grouped<false>(l, d_rowptr, val, x, y, flags, s);
  return e == hipSuccess ? 0 : hip_error(err, -6, "spmv launch", e);
}

}  // namespace gn
