// quant_row.h - the per-row int8 quantizer's arithmetic, shared by the
// standalone quantize kernel and the kernels that quantize a row they already
// hold (fused norm / silu_gate epilogues), so every path gives the same bytes.
//
// Contract (src/ops/quant_ops.h:17-21, src/hal/common/gemm_i8.cpp:49-54,
// 132-171, 209-244): amax = max |x|; s = amax > 0 ? max(amax / 127, FLT_MIN) : 1;
// inv = 1 / s (IEEE division, correctly rounded); q = clamp(rne(x * inv), +-127).
// Compile with contraction off so x * inv stays one rounding.
#pragma once

#include <hip/hip_runtime.h>

#include "wave.h"

#include <cfloat>
#include <cstdint>

namespace vla {
namespace hip {


__device__ __forceinline__ float row_scale(float amax) {
    float s = 1.0f;
    if (amax > 0.0f) {
        s = amax / 127.0f;
        s = s > FLT_MIN ? s : FLT_MIN;
    }
    return s;
}

__device__ __forceinline__ int q8(float v, float inv) {
    int q = (int)rintf(v * inv);
    q = q > 127 ? 127 : q;
    q = q < -127 ? -127 : q;
    return q;
}

__device__ __forceinline__ uint32_t q8x4(float4 v, float inv) {
    return (uint32_t)(q8(v.x, inv) & 0xff) | ((uint32_t)(q8(v.y, inv) & 0xff) << 8) |
           ((uint32_t)(q8(v.z, inv) & 0xff) << 16) | ((uint32_t)(q8(v.w, inv) & 0xff) << 24);
}

}  // namespace hip
}  // namespace vla
