// compat_ops.hip — the element-wise matrix operations and the activation backwards of the
// reference bridge (gpu/matrix/matrix.go and gpu/matrix/activation.go call them), as HIP
// kernels for gfx950:
//
//   a + b, a - b, a * b, a / b          perform_mps_matrix_{add,subtract,element_multiply,
//                                         element_divide}   (metal_bridge_matrix.m:172-479)
//   a + broadcast row / column           perform_mps_matrix_add_broadcast (:252-317)
//   x + s, x * s                         perform_mps_matrix_scalar_{add,multiply} (:481-543)
//   activation backward from the output  perform_activation_*_backward
//                                         (metal_bridge_activation.m:54-702)
//
// All of it is HBM-bound streaming work (8 to 12 bytes per element, no reuse): each
// thread handles 16-byte vectors where every pointer is 16-byte aligned, grid-stride over
// the array, a few blocks per CU. Every formula is written as the reference writes it and
// compiled without contraction (fp contract off), so each operation rounds once, as the C
// source reads. Division is IEEE correctly rounded (hipcc's default for fp32 division,
// the v_div_scale / v_div_fmas / v_div_fixup sequence).
#include <algorithm>
#include <climits>

#include "common.h"

#pragma clang fp contract(off)

namespace gn {
namespace {

constexpr int kBlock = 256;
typedef float float4_t __attribute__((ext_vector_type(4)));

long grid_for(long n, long per_thread) {
  return std::max(1L, std::min(8192L, (n / per_thread + kBlock - 1) / kBlock));
}

// ------------------------------------------------------------------ binary element-wise
enum BinOp { kAdd = 0, kSub = 1, kMul = 2, kDiv = 3 };

template <int OP>
__device__ __forceinline__ float bin(float a, float b) {
  if (OP == kAdd) return a + b;
  if (OP == kSub) return a - b;
  if (OP == kMul) return a * b;
  return a / b;
}

// c[i] = a[i] op b[i]. For division, *zero_at receives the lowest i with b[i] == 0 (the
// element at which the reference loop stops, :470-474); it starts at LONG_MAX.
template <int OP, bool VEC>
__global__ void __launch_bounds__(kBlock) binary_kernel(const float *a, const float *b, float *c, long n,
                                                        unsigned long long *zero_at) {
  const long tid = (long)blockIdx.x * kBlock + threadIdx.x, stride = (long)gridDim.x * kBlock;
  long first_zero = LONG_MAX;
  long done = 0;
  if (VEC) {
    const long n4 = n / 4;
    for (long i = tid; i < n4; i += stride) {
      const float4_t x = reinterpret_cast<const float4_t *>(a)[i];
      const float4_t y = reinterpret_cast<const float4_t *>(b)[i];
      float4_t z;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        z[e] = bin<OP>(x[e], y[e]);
        if (OP == kDiv && y[e] == 0.0f) first_zero = min(first_zero, 4 * i + e);
      }
      reinterpret_cast<float4_t *>(c)[i] = z;
    }
    done = n4 * 4;
  }
  for (long i = done + tid; i < n; i += stride) {
    const float y = b[i];
    c[i] = bin<OP>(a[i], y);
    if (OP == kDiv && y == 0.0f) first_zero = min(first_zero, i);
  }
  if (OP == kDiv && first_zero != LONG_MAX) atomicMin(zero_at, (unsigned long long)first_zero);
}

__global__ void set_u64_kernel(unsigned long long *p, unsigned long long v) { *p = v; }

// ------------------------------------------------------------------ broadcast add
// c[i, j] = a[i * sa_r + j * sa_c] + b[i * sb_r + j * sb_c] over an M x N result: a full
// operand has strides (N, 1), a [1, N] row (0, 1), an [M, 1] column (1, 0).
__global__ void __launch_bounds__(kBlock) add_broadcast_kernel(const float *a, long sa_r, long sa_c, const float *b,
                                                               long sb_r, long sb_c, float *c, long M, long N) {
  const long total = M * N;
  for (long k = (long)blockIdx.x * kBlock + threadIdx.x; k < total; k += (long)gridDim.x * kBlock) {
    const long i = k / N, j = k - i * N;
    c[k] = a[i * sa_r + j * sa_c] + b[i * sb_r + j * sb_c];
  }
}

// y[i] += b[i % L] over the flat array: the bias loop of the reference's ForwardFloat16
// (mixed-precision.go:352-354) for a bias of any length L.
__global__ void __launch_bounds__(kBlock) add_cyclic_kernel(float *y, long n, const float *b, long L) {
  for (long k = (long)blockIdx.x * kBlock + threadIdx.x; k < n; k += (long)gridDim.x * kBlock) y[k] += b[k % L];
}

// ------------------------------------------------------------------ scalar
template <bool MUL, bool VEC>
__global__ void __launch_bounds__(kBlock) scalar_kernel(const float *in, float s, float *out, long n) {
  const long tid = (long)blockIdx.x * kBlock + threadIdx.x, stride = (long)gridDim.x * kBlock;
  long done = 0;
  if (VEC) {
    const long n4 = n / 4;
    for (long i = tid; i < n4; i += stride) {
      float4_t v = reinterpret_cast<const float4_t *>(in)[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = MUL ? v[e] * s : v[e] + s;
      reinterpret_cast<float4_t *>(out)[i] = v;
    }
    done = n4 * 4;
  }
  for (long i = done + tid; i < n; i += stride) out[i] = MUL ? in[i] * s : in[i] + s;
}

// ------------------------------------------------------------------ activation backward
// gradIn from the gradient g and the activation OUTPUT y, as the reference's loops compute
// it (metal_bridge_activation.m): codes are the Go ActivationType values.
__device__ __forceinline__ float backward_from_output(int act, float g, float y, float alpha) {
  switch (act) {
    case 0: return y > 0.0f ? g : 0.0f;                      // :77-79
    case 1: return g * y * (1.0f - y);                        // :137-140
    case 2: return g * (1.0f - y * y);                        // :198-201
    case 4: return g * (y > 0.0f ? 1.0f : alpha);             // :425-429
    case 5: return g * (y > 0.0f ? 1.0f : y + alpha);         // :494-506
    case 6: {                                                 // :569-599
      if (fabsf(y) < 1e-8f) return g * 0.5f;
      float x = y;
      for (int it = 0; it < 3; ++it) {
        const float s = 1.0f / (1.0f + expf(-x));
        const float f = x * s - y;
        const float df = s + x * s * (1.0f - s);
        if (fabsf(df) > 1e-8f) x = x - f / df;
      }
      const float s = 1.0f / (1.0f + expf(-x));
      return g * (s + x * s * (1.0f - s));
    }
    case 7: {                                                 // :665-697
      const float k = 0.7978845608028654f, c = 0.044715f;
      float x = y;
      for (int it = 0; it < 3; ++it) {
        const float x3 = x * x * x;
        const float inner = fmaxf(-88.0f, fminf(88.0f, k * (x + c * x3)));
        const float t = tanhf(inner);
        const float f = 0.5f * x * (1.0f + t) - y;
        const float dt = 1.0f - t * t;
        const float di = k * (1.0f + 3.0f * c * x * x);
        const float df = 0.5f * (1.0f + t) + 0.5f * x * dt * di;
        if (fabsf(df) > 1e-8f) x = x - f / df;
      }
      const float x3 = x * x * x;
      const float inner = fmaxf(-88.0f, fminf(88.0f, k * (x + c * x3)));
      const float t = tanhf(inner);
      const float sech2 = 1.0f - t * t;
      const float di = k * (1.0f + 3.0f * c * x * x);
      return g * (0.5f * (1.0f + t) + 0.5f * x * sech2 * di);
    }
    default: return g;
  }
}

template <bool VEC>
__global__ void __launch_bounds__(kBlock) act_backward_out_kernel(const float *gout, const float *y, float *gin,
                                                                  long n, int act, float alpha) {
  const long tid = (long)blockIdx.x * kBlock + threadIdx.x, stride = (long)gridDim.x * kBlock;
  long done = 0;
  if (VEC) {
    const long n4 = n / 4;
    for (long i = tid; i < n4; i += stride) {
      const float4_t g = reinterpret_cast<const float4_t *>(gout)[i];
      const float4_t v = reinterpret_cast<const float4_t *>(y)[i];
      float4_t r;
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = backward_from_output(act, g[e], v[e], alpha);
      reinterpret_cast<float4_t *>(gin)[i] = r;
    }
    done = n4 * 4;
  }
  for (long i = done + tid; i < n; i += stride) gin[i] = backward_from_output(act, gout[i], y[i], alpha);
}

// Softmax backward per row of [rows, cols]: gin = y * (g - dot(g, y)). One block per row
// (grid-stride over rows); the dot product is summed per thread in index order, then over
// the 64 lanes of each wave by a fixed butterfly and over the 4 waves in order, so a given
// shape always sums in the same order. gin may alias g or y: every element is read for
// the dot product before the barrier that precedes the first write.
__global__ void __launch_bounds__(kBlock) softmax_backward_kernel(const float *g, const float *y, float *gin,
                                                                  long rows, long cols) {
  __shared__ float red[kBlock / 64];
  for (long r = blockIdx.x; r < rows; r += gridDim.x) {
    const float *gr = g + r * cols, *yr = y + r * cols;
    float s = 0.0f;
    for (long i = threadIdx.x; i < cols; i += kBlock) s += gr[i] * yr[i];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    const float dot = (red[0] + red[1]) + (red[2] + red[3]);
    float *out = gin + r * cols;
    for (long i = threadIdx.x; i < cols; i += kBlock) out[i] = yr[i] * (gr[i] - dot);
    __syncthreads();  // red is rewritten by the next row
  }
}

hipError_t last() { return hipGetLastError(); }

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

int launch_binary_f32(int op, const float *a, const float *b, float *c, long n, long *first_zero, hipStream_t s,
                      CError *err) {
  if (n < 0) return set_error(err, -1, "element-wise operation: negative size %ld", n);
  if (first_zero) *first_zero = -1;
  if (n == 0) return 0;
  const bool vec = aligned16(a) && aligned16(b) && aligned16(c);
  const unsigned grid = (unsigned)grid_for(n, vec ? 4 : 1);
  unsigned long long *zero_at = nullptr;
  if (op == kDiv) {
    zero_at = static_cast<unsigned long long *>(dev_alloc(sizeof(unsigned long long), err));
    if (!zero_at) return -1;
    hipLaunchKernelGGL(set_u64_kernel, dim3(1), dim3(1), 0, s, zero_at, (unsigned long long)LONG_MAX);
  }
#define GN_BIN(OPV)                                                                             \
  if (vec)                                                                                      \
    hipLaunchKernelGGL((binary_kernel<OPV, true>), dim3(grid), dim3(kBlock), 0, s, a, b, c, n, zero_at); \
  else                                                                                          \
    hipLaunchKernelGGL((binary_kernel<OPV, false>), dim3(grid), dim3(kBlock), 0, s, a, b, c, n, zero_at)
  switch (op) {
    case kAdd: GN_BIN(kAdd); break;
    case kSub: GN_BIN(kSub); break;
    case kMul: GN_BIN(kMul); break;
    case kDiv: GN_BIN(kDiv); break;
    default: return set_error(err, -1, "element-wise operation: unknown operation %d", op);
  }
#undef GN_BIN
  hipError_t e = last();
  if (e != hipSuccess) {
    dev_free(zero_at);
    return hip_error(err, -1, "element-wise launch", e);
  }
  if (zero_at) {
    unsigned long long z = 0;
    const int rc = download(&z, zero_at, sizeof z, s, err);  // waits for the kernel
    dev_free(zero_at);
    if (rc) return rc;
    if (first_zero) *first_zero = z == (unsigned long long)LONG_MAX ? -1 : (long)z;
  }
  return 0;
}

int launch_add_broadcast_f32(const float *a, long sa_r, long sa_c, const float *b, long sb_r, long sb_c, float *c,
                             long M, long N, hipStream_t s, CError *err) {
  if (M < 0 || N < 0) return set_error(err, -1, "broadcast add: negative size");
  if (M == 0 || N == 0) return 0;
  hipLaunchKernelGGL(add_broadcast_kernel, dim3((unsigned)grid_for(M * N, 1)), dim3(kBlock), 0, s, a, sa_r, sa_c, b,
                     sb_r, sb_c, c, M, N);
  hipError_t e = last();
  return e == hipSuccess ? 0 : hip_error(err, -1, "broadcast add launch", e);
}

int launch_add_cyclic_f32(float *y, long n, const float *b, long L, hipStream_t s, CError *err) {
  if (n < 0 || L < 0) return set_error(err, -1, "cyclic bias add: negative size");
  if (n == 0) return 0;
  if (L == 0) return set_error(err, -1, "cyclic bias add: empty bias");
  hipLaunchKernelGGL(add_cyclic_kernel, dim3((unsigned)grid_for(n, 1)), dim3(kBlock), 0, s, y, n, b, L);
  hipError_t e = last();
  return e == hipSuccess ? 0 : hip_error(err, -6, "cyclic bias add launch", e);
}

int launch_scalar_f32(bool mul, const float *in, float scalar, float *out, long n, hipStream_t s, CError *err) {
  if (n < 0) return set_error(err, -1, "scalar operation: negative size %ld", n);
  if (n == 0) return 0;
  const bool vec = aligned16(in) && aligned16(out);
  const dim3 grid((unsigned)grid_for(n, vec ? 4 : 1));
  if (mul && vec)
    hipLaunchKernelGGL((scalar_kernel<true, true>), grid, dim3(kBlock), 0, s, in, scalar, out, n);
  else if (mul)
    hipLaunchKernelGGL((scalar_kernel<true, false>), grid, dim3(kBlock), 0, s, in, scalar, out, n);
  else if (vec)
    hipLaunchKernelGGL((scalar_kernel<false, true>), grid, dim3(kBlock), 0, s, in, scalar, out, n);
  else
    hipLaunchKernelGGL((scalar_kernel<false, false>), grid, dim3(kBlock), 0, s, in, scalar, out, n);
  hipError_t e = last();
  return e == hipSuccess ? 0 : hip_error(err, -1, "scalar operation launch", e);
}

int launch_act_backward_from_output(const float *gout, const float *y, float *gin, long n, int act, float alpha,
                                    hipStream_t s, CError *err) {
  if (n < 0) return set_error(err, -1, "activation backward: negative size %ld", n);
  if (!(act == 0 || act == 1 || act == 2 || (act >= 4 && act <= 7)))
    return set_error(err, -1, "activation backward: unsupported activation %d", act);
  if (n == 0) return 0;
  const bool vec = aligned16(gout) && aligned16(y) && aligned16(gin);
  const dim3 grid((unsigned)grid_for(n, vec ? 4 : 1));
  if (vec)
    hipLaunchKernelGGL((act_backward_out_kernel<true>), grid, dim3(kBlock), 0, s, gout, y, gin, n, act, alpha);
  else
    hipLaunchKernelGGL((act_backward_out_kernel<false>), grid, dim3(kBlock), 0, s, gout, y, gin, n, act, alpha);
  hipError_t e = last();
  return e == hipSuccess ? 0 : hip_error(err, -1, "activation backward launch", e);
}

int launch_softmax_backward(const float *g, const float *y, float *gin, long rows, long cols, hipStream_t s,
                            CError *err) {
  if (rows < 0 || cols < 0) return set_error(err, -1, "softmax backward: negative size");
  if (rows == 0 || cols == 0) return 0;
  hipLaunchKernelGGL(softmax_backward_kernel, dim3((unsigned)std::min(rows, 65536L)), dim3(kBlock), 0, s, g, y, gin,
                     rows, cols);
  hipError_t e = last();
  return e == hipSuccess ? 0 : hip_error(err, -1, "softmax backward launch", e);
}

}  // namespace gn
