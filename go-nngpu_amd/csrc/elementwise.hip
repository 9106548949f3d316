// elementwise.hip — bandwidth-bound helpers: fp32<->fp16 casts, LDS-tiled
// transpose, synthetic-data generators and a flag-clearing kernel.
#include <algorithm>

#include "act.h"
#include "common.h"

namespace gn {
namespace {

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

unsigned grid_for(size_t work_items, unsigned block) {
  size_t g = (work_items + block - 1) / block;
  const size_t cap = 256u * 32u;  // 32 workgroups per CU on 256 CUs, grid-stride beyond
  if (g > cap) g = cap;
  if (g == 0) g = 1;
  return (unsigned)g;
}

// ------------------------------------------------------------------ casts
// Float32ToFloatMP16 semantics (gpu/matrix/mixed-precision.go:106-151): truncation,
// fp32 subnormal -> signed zero, exponent overflow -> inf, NaN -> 0x7C00 | mant>>13.
__device__ __forceinline__ uint32_t f16_rtz_ref(uint32_t bits) {
  const uint32_t sign = (bits >> 31) << 15;
  const uint32_t exp = (bits >> 23) & 0xFFu;
  uint32_t mant = bits & 0x7FFFFFu;
  if (exp == 0) return sign;
  if (exp == 0xFF) return sign | 0x7C00u | (mant >> 13);
  const int e = (int)exp - 112;  // exp - 127 + 15
  if (e >= 31) return sign | 0x7C00u;
  if (e <= 0) {
    if (e < -10) return sign;
    mant = (mant | 0x800000u) >> (uint32_t)(1 - e);
    return sign | (mant >> 13);
  }
  return sign | ((uint32_t)e << 10) | (mant >> 13);
}

__device__ __forceinline__ uint32_t f16_rne(float x) {
  const _Float16 h = (_Float16)x;  // v_cvt_f16_f32, round-to-nearest-even mode
  return __builtin_bit_cast(uint16_t, h);
}

// The 16-byte load is taken as raw bits; each element is copied into a scalar
// before any bit reinterpretation (a bit cast applied directly to a vector-element
// lvalue reads the vector's first element, whatever the index).
template <int MODE>
__global__ void cast_f32_f16_vec(const u32x4_t *__restrict__ in, u32x2_t *__restrict__ out, size_t n4) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x) {
    const u32x4_t v = in[i];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = MODE ? f16_rtz_ref(w[e]) : f16_rne(__builtin_bit_cast(float, w[e]));
    out[i] = u32x2_t{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
  }
}

template <int MODE>
__global__ void cast_f32_f16_scalar(const float *__restrict__ in, uint16_t *__restrict__ out, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = (uint16_t)(MODE ? f16_rtz_ref(__builtin_bit_cast(uint32_t, in[i])) : f16_rne(in[i]));
}

__global__ void cast_f16_f32_kernel(const uint16_t *__restrict__ in, float *__restrict__ out, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = (float)__builtin_bit_cast(_Float16, in[i]);  // exact widening
}

// ------------------------------------------------------------------ transpose
// 64x64 tiles through LDS (row pitch 65 floats: column reads hit distinct banks).
__global__ void __launch_bounds__(256) transpose_kernel(const float *__restrict__ in, long rows, long cols,
                                                        float *__restrict__ out) {
  __shared__ float tile[64][65];
  const long tiles_c = (cols + 63) / 64;
  const long r0 = (long)(blockIdx.x / tiles_c) * 64;
  const long c0 = (long)(blockIdx.x % tiles_c) * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int r = ty + 4 * k;
    if (r0 + r < rows && c0 + tx < cols) tile[r][tx] = in[(r0 + r) * cols + c0 + tx];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int c = ty + 4 * k;  // output row = input column
    if (c0 + c < cols && r0 + tx < rows) out[(c0 + c) * rows + r0 + tx] = tile[tx][c];
  }
}

// ------------------------------------------------------------------ generators
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

__global__ void fill_uniform_kernel(float *out, size_t n, uint64_t base, float lo, float hi) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const double u = (double)(mix64(base + (i + 1) * 0x9E3779B97F4A7C15ULL) >> 40) * (1.0 / 16777216.0);
    out[i] = (float)((double)lo + ((double)hi - (double)lo) * u);
  }
}

__global__ void fill_normal_kernel(float *out, size_t n, uint64_t base, float mean, float sd) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const uint64_t a = mix64(base + (2 * i + 1) * 0x9E3779B97F4A7C15ULL);
    const uint64_t b = mix64(base + (2 * i + 2) * 0x9E3779B97F4A7C15ULL);
    const double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);
    const double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
    const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925286766559 * u2);
    out[i] = (float)((double)mean + (double)sd * z);
  }
}

__global__ void zero_i32_kernel(int *p, long n) {
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) p[i] = 0;
}

uint64_t stream_base(uint64_t seed, uint64_t sid) {
  uint64_t z = sid + 0x632BE59BD9B4E019ULL;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return seed ^ (z ^ (z >> 31));
}

// ------------------------------------------------------------------ activation backward
// Derivative of the activations of act.h (apply_act, Go ActivationType codes)
// with respect to their input x, evaluated at x.
__device__ __forceinline__ float act_grad(int act, float x, float a) {
  switch (act) {
    case 0: return x > 0.0f ? 1.0f : 0.0f;
    case 1: {
      const float sg = 1.0f / (1.0f + __expf(-fmaxf(-88.0f, fminf(88.0f, x))));
      return sg * (1.0f - sg);
    }
    case 2: {
      const float t = tanhf(x);
      return 1.0f - t * t;
    }
    case 4: return x > 0.0f ? 1.0f : a;
    case 5: return x > 0.0f ? 1.0f : a * __expf(fmaxf(-88.0f, x));
    case 6: {
      const float c = fmaxf(-88.0f, fminf(88.0f, x));
      const float sg = 1.0f / (1.0f + __expf(-c));
      return sg + c * sg * (1.0f - sg);
    }
    case 7: {
      const float k = 0.7978845608028654f;
      const float inner = fmaxf(-88.0f, fminf(88.0f, k * (x + 0.044715f * x * x * x)));
      const float t = tanhf(inner);
      return 0.5f * (1.0f + t) + 0.5f * x * (1.0f - t * t) * k * (1.0f + 3.0f * 0.044715f * x * x);
    }
    default: return 1.0f;
  }
}

// One thread per column j and chunk of R rows (blockIdx.y): grad_in = (grad_out * act') *
// scale, and partial[chunk, j] = the chunk's column sum in row order. A wave's 64
// threads read 64 consecutive columns of a row: one coalesced 256-byte segment.
__global__ void __launch_bounds__(256) act_backward_kernel(const float *__restrict__ dy, const float *__restrict__ pre,
                                                           long M, long N, int act, float alpha, float scale,
                                                           float *dx, float *__restrict__ partial, long R) {
  const long j = (long)blockIdx.x * 256 + threadIdx.x;
  if (j >= N) return;
  const long r0 = (long)blockIdx.y * R;
  const long r1 = min(M, r0 + R);
  float sum = 0.0f;
  for (long r = r0; r < r1; ++r) {
    const long i = r * N + j;
    const float g = (dy[i] * act_grad(act, pre[i], alpha)) * scale;
    dx[i] = g;
    sum += g;
  }
  if (partial) partial[(long)blockIdx.y * N + j] = sum;
}

// ------------------------------------------------------------------ activation forward
// y = act(x) element-wise (act.h, precise math). VEC: in and out are 16-byte aligned and
// n4 float4 groups are processed as vectors; the n % 4 tail is done by the first lanes.
template <bool VEC>
__global__ void __launch_bounds__(256) act_forward_kernel(const float *__restrict__ in, float *__restrict__ out,
                                                          size_t n, int act, float alpha) {
  const size_t tid = (size_t)blockIdx.x * 256 + threadIdx.x, stride = (size_t)gridDim.x * 256;
  size_t done = 0;
  if (VEC) {
    const size_t n4 = n / 4;
    for (size_t i = tid; i < n4; i += stride) {
      float4_t v = reinterpret_cast<const float4_t *>(in)[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = apply_act<false>(act, v[e], alpha);
      reinterpret_cast<float4_t *>(out)[i] = v;
    }
    done = n4 * 4;
  }
  for (size_t i = done + tid; i < n; i += stride) out[i] = apply_act<false>(act, in[i], alpha);
}

// Sum (MAX = false) or maximum (MAX = true) over the 256 threads of a block; every
// thread gets the result. red holds 4 floats of LDS.
template <bool MAX>
__device__ __forceinline__ float block_reduce(float v, float *red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float w = __shfl_xor(v, o, 64);
    v = MAX ? fmaxf(v, w) : v + w;
  }
  __syncthreads();  // red is reused by consecutive reductions
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return MAX ? fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])) : (red[0] + red[1]) + (red[2] + red[3]);
}

// Row-wise softmax of a [rows, cols] matrix, one 256-thread block per row (grid-stride
// over rows): m = max of the row (fmaxf, so NaNs are skipped as in the reference),
// s = sum of expf(x - m), y = expf(x - m) / s. The reference's loops
// (metal_bridge_activation.m:206-242, :283-325) compute the same per element; only the
// order of the sum differs.
__global__ void __launch_bounds__(256) softmax_rows_kernel(const float *__restrict__ in, float *__restrict__ out,
                                                           long rows, long cols) {
  __shared__ float red[4];
  for (long r = blockIdx.x; r < rows; r += gridDim.x) {
    const float *x = in + r * cols;
    float *y = out + r * cols;
    float m = -INFINITY;
    for (long i = threadIdx.x; i < cols; i += 256) m = fmaxf(m, x[i]);
    m = block_reduce<true>(m, red);
    float sum = 0.0f;
    for (long i = threadIdx.x; i < cols; i += 256) sum += expf(x[i] - m);
    sum = block_reduce<false>(sum, red);
    for (long i = threadIdx.x; i < cols; i += 256) y[i] = expf(x[i] - m) / sum;
  }
}

// out[j] = sum of partial[c, j] over c = 0, 1, ... (fixed order: deterministic).
__global__ void __launch_bounds__(256) colsum_finish_kernel(const float *__restrict__ partial, long chunks, long N,
                                                            float *__restrict__ out) {
  const long j = (long)blockIdx.x * 256 + threadIdx.x;
  if (j >= N) return;
  float sum = 0.0f;
  for (long c = 0; c < chunks; ++c) sum += partial[c * N + j];
  out[j] = sum;
}

}  // namespace

bool act_grad_supported(int act) { return act == -1 || act == 0 || act == 1 || act == 2 || (act >= 4 && act <= 7); }

namespace {

// Work split of the activation backward: (column block of 256, row chunk) workgroups, enough
// of them to fill the GPU with at least 8 rows each. The column sums are added over the
// chunks in a fixed order, so a given (rows, cols) always sums in the same order.
struct ActBackwardPlan {
  long colblocks, chunks, R;
};

int plan_act_backward(long rows, long cols, ActBackwardPlan &pl, CError *err) {
  pl.colblocks = (cols + 255) / 256;
  if (pl.colblocks > 0x7FFFFFFFL) return set_error(err, -1, "activation backward: too many columns");
  long chunks = (4096 + pl.colblocks - 1) / pl.colblocks;
  chunks = std::max(1L, std::min(chunks, (rows + 7) / 8));
  pl.R = (rows + chunks - 1) / chunks;
  pl.chunks = (rows + pl.R - 1) / pl.R;
  return 0;
}

// Common argument checks; 1 when there is nothing to compute beyond the empty column sum.
int check_act_backward(const float *grad_out, const float *pre, long rows, long cols, int act, float *grad_in,
                       CError *err) {
  if (rows < 0 || cols < 0) return set_error(err, -1, "activation backward: negative size");
  if (!act_grad_supported(act)) return set_error(err, -1, "activation backward: unsupported activation %d", act);
  if (cols == 0 || rows == 0) return 1;
  if (!grad_out || !pre || !grad_in) return set_error(err, -1, "activation backward: NULL pointer");
  return 0;
}

// An empty column sum is zero: a kernel, not a memset, so it can be captured.
int zero_bias(long cols, float *grad_bias, hipStream_t s, CError *err) {
  if (!grad_bias || cols == 0) return 0;
  hipLaunchKernelGGL(colsum_finish_kernel, dim3((unsigned)((cols + 255) / 256)), dim3(256), 0, s, nullptr, 0L, cols,
                     grad_bias);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : hip_error(err, -6, "activation backward launch", e);
}

// The two kernels of the backward: element-wise gradient (plus per-chunk column sums into
// `partial`, chunks x cols floats, when grad_bias is wanted), then the fixed-order sum.
int enqueue_act_backward(const ActBackwardPlan &pl, const float *grad_out, const float *pre, long rows, long cols,
                         int act, float alpha, float scale, float *grad_in, float *grad_bias, float *partial,
                         hipStream_t s, CError *err) {
  hipLaunchKernelGGL(act_backward_kernel, dim3((unsigned)pl.colblocks, (unsigned)pl.chunks), dim3(256), 0, s, grad_out,
                     pre, rows, cols, act, alpha, scale, grad_in, grad_bias ? partial : nullptr, pl.R);
  if (grad_bias)
    hipLaunchKernelGGL(colsum_finish_kernel, dim3((unsigned)pl.colblocks), dim3(256), 0, s, partial, pl.chunks, cols,
                       grad_bias);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : hip_error(err, -6, "activation backward launch", e);
}

// ------------------------------------------------------------------ allocation-free variant
// Scratch of gn_activation_backward_noalloc: the per-chunk column sums live in this
// file-scope device array instead of library-allocated memory. Each device the library runs
// on holds its own copy (kNoAllocScratchBytes) until the process ends; calls on one device
// share it, so calls that overlap on one device race. Host code never passes `scratch`
// itself to a kernel (in host code the name is a stand-in, not a device address): it uses
// the address hipGetSymbolAddress returns for the current device, kept per device below.
constexpr size_t kNoAllocScratchFloats = size_t(1) << 21;  // 8 MiB
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
float *g_noalloc_ptr[kMaxDevices] = {};

// Address of `scratch` on the current device (looked up once per device).
float *noalloc_scratch(CError *err) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    hip_error(err, -1, "activation backward (no-alloc): hipGetDevice", e);
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_error(err, -1, "activation backward (no-alloc): device %d beyond the %d supported", dev, kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if (!g_noalloc_ptr[dev]) {
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      hip_error(err, -1, "activation backward (no-alloc): hipGetSymbolAddress(scratch)", e);
      return nullptr;
    }
    g_noalloc_ptr[dev] = static_cast<float *>(ptr);
  }
  return g_noalloc_ptr[dev];
}

}  // namespace

int noalloc_scratch_setup(CError *err) { return noalloc_scratch(err) ? 0 : -1; }

int launch_act_backward(const float *grad_out, const float *pre, long rows, long cols, int act, float alpha,
                        float scale, float *grad_in, float *grad_bias, hipStream_t s, CError *err) {
  if (int rc = check_act_backward(grad_out, pre, rows, cols, act, grad_in, err))
    return rc < 0 ? rc : zero_bias(cols, grad_bias, s, err);
  ActBackwardPlan pl;
  if (int rc = plan_act_backward(rows, cols, pl, err)) return rc;
  float *partial = nullptr;
  std::unique_lock<std::mutex> lk;
  if (grad_bias) {
    partial = static_cast<float *>(stream_scratch(s, (size_t)pl.chunks * (size_t)cols * sizeof(float), lk, err));
    if (!partial) return -3;
  }
  return enqueue_act_backward(pl, grad_out, pre, rows, cols, act, alpha, scale, grad_in, grad_bias, partial, s, err);
}

int launch_act_backward_noalloc(const float *grad_out, const float *pre, long rows, long cols, int act, float alpha,
                                float scale, float *grad_in, float *grad_bias, hipStream_t s, CError *err) {
  if (int rc = check_act_backward(grad_out, pre, rows, cols, act, grad_in, err))
    return rc < 0 ? rc : zero_bias(cols, grad_bias, s, err);
  ActBackwardPlan pl;
  if (int rc = plan_act_backward(rows, cols, pl, err)) return rc;
  float *partial = nullptr;
  if (grad_bias) {
    const size_t need = (size_t)pl.chunks * (size_t)cols;
    if (need > kNoAllocScratchFloats)
      return set_error(err, -1,
                       "activation backward (no-alloc): %ld columns need %zu floats of partial sums, more than the "
                       "%zu-float scratch (at most %zu columns)",
                       cols, need, kNoAllocScratchFloats, kNoAllocScratchFloats);
    partial = noalloc_scratch(err);
    if (!partial) return -1;
  }
  return enqueue_act_backward(pl, grad_out, pre, rows, cols, act, alpha, scale, grad_in, grad_bias, partial, s, err);
}

bool act_forward_supported(int act) { return act == -1 || act == 0 || act == 1 || act == 2 || (act >= 4 && act <= 7); }

int launch_act_forward(const float *in, float *out, long n, int act, float alpha, hipStream_t s, CError *err) {
  if (n < 0) return set_error(err, -1, "activation forward: negative size %ld", n);
  if (!act_forward_supported(act)) return set_error(err, -1, "activation forward: unsupported activation %d", act);
  if (n == 0) return 0;
  const bool vec = (((uintptr_t)in | (uintptr_t)out) & 15) == 0;
  const long per = vec ? 4 : 1;
  const long blocks = std::max(1L, std::min(8192L, (n / per + 255) / 256));
  if (vec)
    hipLaunchKernelGGL(act_forward_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, in, out, (size_t)n, act, alpha);
  else
    hipLaunchKernelGGL(act_forward_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s, in, out, (size_t)n, act, alpha);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : hip_error(err, -1, "activation forward launch", e);
}

int launch_softmax_rows(const float *in, float *out, long rows, long cols, hipStream_t s, CError *err) {
  if (rows < 0 || cols < 0) return set_error(err, -1, "softmax: negative size");
  if (rows == 0 || cols == 0) return 0;
  const long blocks = std::min(rows, 65536L);
  hipLaunchKernelGGL(softmax_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, s, in, out, rows, cols);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : hip_error(err, -1, "softmax launch", e);
}

int launch_cast_f32_f16(const float *in, uint16_t *out, size_t n, int mode, hipStream_t s, CError *err) {
  if (mode != GN_ROUND_NEAREST_EVEN && mode != GN_ROUND_TOWARD_ZERO)
    return set_error(err, -1, "cast: unknown rounding mode %d", mode);
  if (n == 0) return 0;
  if (!in || !out) return set_error(err, -1, "cast: NULL pointer");
  const bool vec = (n % 4 == 0) && ((uintptr_t)in % 16 == 0) && ((uintptr_t)out % 8 == 0);
  if (vec) {
    const size_t n4 = n / 4;
    if (mode) hipLaunchKernelGGL(cast_f32_f16_vec<1>, dim3(grid_for(n4, 256)), dim3(256), 0, s,
                                 (const u32x4_t *)in, (u32x2_t *)out, n4);
    else hipLaunchKernelGGL(cast_f32_f16_vec<0>, dim3(grid_for(n4, 256)), dim3(256), 0, s,
                            (const u32x4_t *)in, (u32x2_t *)out, n4);
  } else {
    if (mode) hipLaunchKernelGGL(cast_f32_f16_scalar<1>, dim3(grid_for(n, 256)), dim3(256), 0, s, in, out, n);
    else hipLaunchKernelGGL(cast_f32_f16_scalar<0>, dim3(grid_for(n, 256)), dim3(256), 0, s, in, out, n);
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : hip_error(err, -6, "cast launch", e);
}

int launch_cast_f16_f32(const uint16_t *in, float *out, size_t n, hipStream_t s, CError *err) {
  if (n == 0) return 0;
  if (!in || !out) return set_error(err, -1, "cast: NULL pointer");
  hipLaunchKernelGGL(cast_f16_f32_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, in, out, n);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : hip_error(err, -6, "cast launch", e);
}

int launch_transpose_f32(const float *in, long rows, long cols, float *out, hipStream_t s, CError *err) {
  if (rows < 0 || cols < 0) return set_error(err, -1, "transpose: negative size");
  if (rows == 0 || cols == 0) return 0;
  if (!in || !out) return set_error(err, -1, "transpose: NULL pointer");
  const long tiles = ((rows + 63) / 64) * ((cols + 63) / 64);
  if (tiles > 0x7FFFFFFFL) return set_error(err, -1, "transpose: too large");
  hipLaunchKernelGGL(transpose_kernel, dim3((unsigned)tiles), dim3(256), 0, s, in, rows, cols, out);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : hip_error(err, -6, "transpose launch", e);
}

int launch_fill_uniform(float *out, size_t n, uint64_t seed, uint64_t sid, float lo, float hi, hipStream_t s,
                        CError *err) {
  if (n == 0) return 0;
  if (!out) return set_error(err, -1, "fill: NULL pointer");
  hipLaunchKernelGGL(fill_uniform_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, out, n, stream_base(seed, sid),
                     lo, hi);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : hip_error(err, -6, "fill launch", e);
}

int launch_fill_normal(float *out, size_t n, uint64_t seed, uint64_t sid, float mean, float sd, hipStream_t s,
                       CError *err) {
  if (n == 0) return 0;
  if (!out) return set_error(err, -1, "fill: NULL pointer");
  hipLaunchKernelGGL(fill_normal_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, out, n, stream_base(seed, sid),
                     mean, sd);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : hip_error(err, -6, "fill launch", e);
}

int launch_zero_i32(int *p, long n, hipStream_t s, CError *err) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(zero_i32_kernel, dim3(1), dim3(64), 0, s, p, n);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : hip_error(err, -6, "zero launch", e);
}

}  // namespace gn
