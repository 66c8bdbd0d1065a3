// act.h - elementwise activations shared by the GEMM epilogue and the
// standalone eltwise kernels, so a fused epilogue and the separate pass give
// the same values.
//
// Formulas are the reference's scalar forms (src/hal/common/eltwise.cpp):
//   relu       x < 0 ? 0 : x                       (:209-215; -0 stays -0)
//   gelu_tanh  0.5 x (1 + tanh(c (x + 0.044715 x^3))), c = sqrt(2/pi)  (:120-127)
//   gelu_erf   0.5 x (1 + erf(x / sqrt 2))          (:200-206)
//   silu_gate  (g / (1 + exp(-g))) * u              (:58-63)
//   silu       x / (1 + exp(-x))                    (:66-72)
// evaluated with ROCm's device libm (tanhf, erff, expf). The reference's SIMD
// paths replace tanh/erf/exp with Cephes-style polynomials; both sit within
// the tests' 2e-6 relative class of the double-precision formula.
#pragma once

#include <hip/hip_runtime.h>

namespace vla {
namespace hip {

__device__ __forceinline__ float act_relu(float v) { return v < 0.0f ? 0.0f : v; }
// The ReLU of ResNet's residual add (x > 0 ? x : 0: -0 and NaN give +0),
// shared by the add + ReLU pass and the conv epilogue that fuses it.
__device__ __forceinline__ float relu_gt(float v) { return v > 0.0f ? v : 0.0f; }

__device__ __forceinline__ float act_gelu_tanh(float v) {
    const float c = 0.7978845608028654f;
    return 0.5f * v * (1.0f + tanhf(c * (v + 0.044715f * v * v * v)));
}

__device__ __forceinline__ float act_gelu_erf(float v) {
    const float inv_sqrt2 = 0.70710678118654752f;
    return 0.5f * v * (1.0f + erff(v * inv_sqrt2));
}

__device__ __forceinline__ float act_silu_gate(float g, float u) {
    return (g / (1.0f + expf(-g))) * u;
}

// x / (1 + exp(-x)): the SiLU of action_time_mlp_in
// (src/models/smolvla/action_expert.cpp:209)
__device__ __forceinline__ float act_silu(float v) { return v / (1.0f + expf(-v)); }

// act: 0 none, 1 relu, 2 gelu_tanh, 3 gelu_erf, 4 silu (vla_act)
template <int ACT>
__device__ __forceinline__ float apply_act(float v) {
    if (ACT == 1) return act_relu(v);
    if (ACT == 2) return act_gelu_tanh(v);
    if (ACT == 3) return act_gelu_erf(v);
    if (ACT == 4) return act_silu(v);
    return v;
}

}  // namespace hip
}  // namespace vla
