// mfma_ceiling — the sustained rate of the fp16 matrix instructions with operands held in
// registers: no LDS, no memory traffic, so nothing but the MFMA pipe and the chip's clock
// bounds it. Two instructions of equal nominal peak are measured in the same process:
//   v_mfma_f32_16x16x32_f16  (16 384 flop, 2 KiB of A+B operands per wave instruction)
//   v_mfma_f32_32x32x16_f16  (32 768 flop, the same 2 KiB: half the operand bytes per flop)
// Each wave keeps independent accumulators (16 of 16x16, or 8 of 32x32: 64 or 128
// accumulator registers) and cycles through four A and four B fragments (loaded once), so
// the multiplier inputs change with every instruction, as in a GEMM. Workgroups of 4 waves,
// two per CU (two waves per SIMD, as in the 256 x 256 GEMM tiles).
//
// The operand values set the power drawn, and under a board power limit the clock follows:
// "gemm" data has the C3 benchmark's distributions (A ~ N(0,1), B ~ N(0, 0.02^2), rounded to
// fp16), "zero" data has every operand 0. The gap between the two is the power limit's cost;
// the "gemm" rate is the ceiling a GEMM on such data can reach with that instruction.
//
// Usage: mfma_ceiling [seconds per data set and instruction, default 3]. Prints one JSON
// object: the 16x16x32 figures at top level ("gemm_data", "zero_data") and the 32x32x16
// figures under "mfma_32x32x16".
#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <vector>

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int kBlocks = 512;   // 2 per CU on 256 CUs
constexpr int kThreads = 256;  // 4 waves
constexpr int kMfmaPerIter = 16;

// 16 instructions per iteration, each on its own 16x16 accumulator.
__global__ void __launch_bounds__(kThreads) mfma16_loop(const half8_t *src, float *out, int iters) {
  const int lane = threadIdx.x & 63;
  const long base = (long)blockIdx.x * 8 * 64;
  half8_t a[4], b[4];
  for (int i = 0; i < 4; ++i) {
    a[i] = src[base + i * 64 + lane];
    b[i] = src[base + (4 + i) * 64 + lane];
  }
  float4_t acc[kMfmaPerIter];
  for (int i = 0; i < kMfmaPerIter; ++i) acc[i] = float4_t{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < kMfmaPerIter; ++i)
      acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i & 3], b[(i >> 2) & 3], acc[i], 0, 0, 0);
  }
  float s = 0.f;
  for (int i = 0; i < kMfmaPerIter; ++i) s += acc[i][0] + acc[i][1] + acc[i][2] + acc[i][3];
  out[blockIdx.x * kThreads + threadIdx.x] = s;  // keeps the loop live
}

// 16 instructions per iteration over 8 accumulators of 32x32 (each updated twice, 7
// instructions apart, beyond the instruction's 16-pass latency).
__global__ void __launch_bounds__(kThreads) mfma32_loop(const half8_t *src, float *out, int iters) {
  const int lane = threadIdx.x & 63;
  const long base = (long)blockIdx.x * 8 * 64;
  half8_t a[4], b[4];
  for (int i = 0; i < 4; ++i) {
    a[i] = src[base + i * 64 + lane];
    b[i] = src[base + (4 + i) * 64 + lane];
  }
  float16_t acc[8];
  for (int i = 0; i < 8; ++i)
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < kMfmaPerIter; ++i)
      acc[i & 7] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i & 3], b[(i >> 2) & 3], acc[i & 7], 0, 0, 0);
  }
  float s = 0.f;
  for (int i = 0; i < 8; ++i)
    for (int e = 0; e < 16; ++e) s += acc[i][e];
  out[blockIdx.x * kThreads + threadIdx.x] = s;
}

static void check(hipError_t e, const char *what) {
  if (e != hipSuccess) {
    std::fprintf(stderr, "mfma_ceiling: %s: %s\n", what, hipGetErrorString(e));
    std::exit(1);
  }
}

struct Rate {
  double tflops, ms;
  int launches;
};

static Rate measure(bool wide, const half8_t *src, float *out, double seconds, hipEvent_t e0, hipEvent_t e1) {
  const int iters = wide ? 10000 : 20000;  // equal flop per launch
  const double flop_per_mfma = wide ? 32.0 * 32.0 * 16.0 * 2.0 : 16.0 * 16.0 * 32.0 * 2.0;
  const double flop = (double)kBlocks * (kThreads / 64) * iters * kMfmaPerIter * flop_per_mfma;
  auto launch = [&]() {
    if (wide)
      hipLaunchKernelGGL(mfma32_loop, dim3(kBlocks), dim3(kThreads), 0, 0, src, out, iters);
    else
      hipLaunchKernelGGL(mfma16_loop, dim3(kBlocks), dim3(kThreads), 0, 0, src, out, iters);
  };
  for (int w = 0; w < 3; ++w) launch();
  check(hipDeviceSynchronize(), "warm-up");
  double total_ms = 0.0;
  int n = 0;
  const auto t0 = std::chrono::steady_clock::now();
  while (std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() < seconds) {
    check(hipEventRecord(e0, 0), "hipEventRecord");
    launch();
    check(hipEventRecord(e1, 0), "hipEventRecord");
    check(hipEventSynchronize(e1), "hipEventSynchronize");
    float ms = 0.f;
    check(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
    total_ms += ms;
    ++n;
  }
  return Rate{flop / (total_ms / n) / 1e9, total_ms / n, n};
}

int main(int argc, char **argv) {
  const double seconds = argc > 1 ? std::atof(argv[1]) : 3.0;
  const size_t nvec = (size_t)kBlocks * 8 * 64;  // half8 fragments: 4 A and 4 B per wave lane set
  half8_t *src = nullptr;
  float *out = nullptr;
  check(hipMalloc(&src, nvec * sizeof(half8_t)), "hipMalloc");
  check(hipMalloc(&out, (size_t)kBlocks * kThreads * sizeof(float)), "hipMalloc");
  hipEvent_t e0, e1;
  check(hipEventCreate(&e0), "hipEventCreate");
  check(hipEventCreate(&e1), "hipEventCreate");
  Rate r[2][2];  // [data set][instruction]
  for (int set = 0; set < 2; ++set) {
    std::vector<_Float16> h(nvec * 8);
    unsigned x = 12345u;
    auto uni = [&x]() {
      x = x * 1664525u + 1013904223u;
      return ((x >> 8) + 0.5f) / 16777216.0f;
    };
    for (size_t i = 0; i < h.size(); ++i) {
      // within each wave's 8 fragments, the first 4 are A, the last 4 B
      const bool is_b = (i / (64 * 8)) % 8 >= 4;
      const float z = std::sqrt(-2.0f * std::log(uni())) * std::cos(6.2831853f * uni());  // N(0,1)
      h[i] = set == 0 ? (_Float16)(is_b ? 0.02f * z : z) : (_Float16)0.0f;
    }
    check(hipMemcpy(src, h.data(), nvec * sizeof(half8_t), hipMemcpyHostToDevice), "hipMemcpy");
    for (int wide = 0; wide < 2; ++wide) r[set][wide] = measure(wide != 0, src, out, seconds, e0, e1);
  }
  auto pr = [](const char *key, const Rate &q, bool comma) {
    std::printf("\"%s\": {\"tflops\": %.1f, \"launches\": %d, \"ms_per_launch\": %.3f}%s", key, q.tflops,
                q.launches, q.ms, comma ? ", " : "");
  };
  std::printf("{\"instruction\": \"v_mfma_f32_16x16x32_f16\", \"workgroups\": %d, \"waves_per_simd\": 2, ", kBlocks);
  pr("gemm_data", r[0][0], true);
  pr("zero_data", r[1][0], true);
  std::printf("\"mfma_32x32x16\": {\"instruction\": \"v_mfma_f32_32x32x16_f16\", ");
  pr("gemm_data", r[0][1], true);
  pr("zero_data", r[1][1], false);
  std::printf("}}\n");
  check(hipFree(src), "hipFree");
  check(hipFree(out), "hipFree");
  return 0;
}
