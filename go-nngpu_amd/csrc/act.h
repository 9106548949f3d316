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
      float inner = 0.7978845608028654f * (x + 0.044715f * x * x * x);
      inner = fmaxf(-88.0f, fminf(88.0f, inner));
      if (!FAST) return 0.5f * x * (1.0f + tanhf(inner));
      // 0.5 (1 + tanh(u)) = 1 / (1 + e^(-2u)): one exp and one reciprocal, no
      // cancellation near u = 0, and the clamped limits are exact (e^(-2u) underflows
      // to 0 at u = 88, giving x; it overflows to inf at u = -88, giving x * 0).
      return x * inv(1.0f + __expf(-2.0f * inner));
    }
    default: return x;
  }
}

}  // namespace gn
