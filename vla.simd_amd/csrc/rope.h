// rope.h - the NeoX rotation of one pair (x0, x1) = (x[i], x[i + half]) of a
// head with that token's (cos, sin) of pair i (rope_neox,
// src/hal/common/norms.cpp:37-67): x0' = x0 cos - x1 sin, x1' = x0 sin +
// x1 cos, evaluated in double and rounded once to float. The fused
// multiply-adds are written out, so every kernel that rotates - the RoPE
// kernels and the skinny GEMM's rotating epilogue - gives the same floats
// whatever contraction its translation unit compiles with.
#pragma once

#include <hip/hip_runtime.h>

namespace vla {
namespace hip {

__device__ __forceinline__ float rope_lo(float x0, float x1, double c, double s) {
    return (float)__builtin_fma((double)x0, c, -((double)x1 * s));
}

__device__ __forceinline__ float rope_hi(float x0, float x1, double c, double s) {
    return (float)__builtin_fma((double)x0, s, (double)x1 * c);
}

}  // namespace hip
}  // namespace vla
