// act.h — element-wise activations shared by the GEMM epilogue and the stand-alone
// activation kernels. Codes are the Go ActivationType values (gpu/matrix/activation.go:
// 20-29); any other code (GN_ACT_NONE = -1) is the identity. The formulas follow the
// reference's forward loops (internal/cgo/metal_bridge_activation.m): Sigmoid, Tanh and
// Swish clamp x to [-88, 88] first (Swish then returns clamped_x * sigmoid(clamped_x)),
// ELU clamps the exp argument at -88, GELU is the tanh form with its inner argument
// clamped to [-88, 88] (:606-639).
#pragma once

#include <hip/hip_runtime.h>

namespace gn {

// FAST (the GEMM epilogue, which runs while the matrix cores idle) uses __expf and the
// hardware reciprocal (v_rcp_f32, 1 ulp) in place of expf and the IEEE divide sequence,
// and GELU's sigmoid form; the stand-alone activation kernels are memory-bound and use
// expf, tanhf and exact division instead.
template <bool FAST = true>
__device__ __forceinline__ float apply_act(int act, float x, float a) {
  auto ex = [](float v) { return FAST ? __expf(v) : expf(v); };
  auto inv = [](float v) { return FAST ? __builtin_amdgcn_rcpf(v) : 1.0f / v; };
  switch (act) {
    case 0: return fmaxf(0.0f, x);
    case 1: { float c = fmaxf(-88.0f, fminf(88.0f, x)); return inv(1.0f + ex(-c)); }
    case 2: return tanhf(fmaxf(-88.0f, fminf(88.0f, x)));
    case 4: return x > 0.0f ? x : a * x;
    case 5: return x > 0.0f ? x : a * (ex(fmaxf(-88.0f, x)) - 1.0f);
    case 6: { float c = fmaxf(-88.0f, fminf(88.0f, x)); return c * inv(1.0f + ex(-c)); }
    case 7: {
      if (!FAST) {
        float inner = 0.7978845608028654f * (x + 0.044715f * x * x * x);
        inner = fmaxf(-88.0f, fminf(88.0f, inner));
        return 0.5f * x * (1.0f + tanhf(inner));
      }
      // 0.5 (1 + tanh(u)) = 1 / (1 + e^(-2u)), u = sqrt(2/pi) (x + 0.044715 x^3): one
      // base-2 exponential and one reciprocal, no cancellation near u = 0. The constants
      // are folded, e^(-2u) = 2^(x (k0 + k1 x^2)) with k0 = -2 sqrt(2/pi) log2(e) and
      // k1 = 0.044715 k0: 5 VALU and 2 transcendental instructions per element. The clamp
      // of u to [-88, 88] needs no instruction here: 2^t saturates as e^(-2u) does at
      // those bounds (to 0 for t < -126, giving x; to inf for t > 128, giving x * 0).
      constexpr float k0 = -2.302208198f, k1 = -0.1029432309f;
      const float t = x * __builtin_fmaf(k1, x * x, k0);
      return x * inv(1.0f + __builtin_amdgcn_exp2f(t));
    }
    default: return x;
  }
}

}  // namespace gn
