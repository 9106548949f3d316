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

// FAST (the GEMM epilogue) uses __expf and GELU's one-exp tanh; the stand-alone
// activation kernels are memory-bound and use expf and tanhf instead.
template <bool FAST = true>
__device__ __forceinline__ float apply_act(int act, float x, float a) {
  auto ex = [](float v) { return FAST ? __expf(v) : expf(v); };
  switch (act) {
    case 0: return fmaxf(0.0f, x);
    case 1: { float c = fmaxf(-88.0f, fminf(88.0f, x)); return 1.0f / (1.0f + ex(-c)); }
    case 2: return tanhf(fmaxf(-88.0f, fminf(88.0f, x)));
    case 4: return x > 0.0f ? x : a * x;
    case 5: return x > 0.0f ? x : a * (ex(fmaxf(-88.0f, x)) - 1.0f);
    case 6: { float c = fmaxf(-88.0f, fminf(88.0f, x)); return c / (1.0f + ex(-c)); }
    case 7: {
      float inner = 0.7978845608028654f * (x + 0.044715f * x * x * x);
      inner = fmaxf(-88.0f, fminf(88.0f, inner));
      if (!FAST) return 0.5f * x * (1.0f + tanhf(inner));
      // tanh(u) = 1 - 2 / (e^(2u) + 1): one exp and one divide instead of tanhf; the
      // limits are exact (e -> 0 gives -1, e -> inf gives +1), and near u = 0 the
      // absolute error stays at fp32 rounding level, far below the GEMM's own.
      const float t = 1.0f - 2.0f / (__expf(2.0f * inner) + 1.0f);
      return 0.5f * x * (1.0f + t);
    }
    default: return x;
  }
}

}  // namespace gn
