// wave.h - wave64 reductions through DPP lane permutations (applied in the
// vector ALU, no LDS round trip per step as ds_bpermute takes), gfx9 / CDNA
// encodings: quad_perm xor 1 and xor 2, row_shr 4 and 8 inside each 16-lane
// row, then row_bcast 15 (rows 1, 3 take the previous row's lane 15) and
// row_bcast 31 (rows 2, 3 take lane 31). Lane 63 then holds the whole-wave
// result, which readlane broadcasts. Lanes a permutation gives no source keep
// the identity, so the tree is the same fixed order on every call.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace vla {
namespace hip {

template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t identity, uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)identity, (int)v, CTRL, ROWS, 0xf, false);
}

template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_f32(float identity, float v) {
    return __uint_as_float(dpp_u32<CTRL, ROWS>(__float_as_uint(identity), __float_as_uint(v)));
}

template <int CTRL, int ROWS>
__device__ __forceinline__ double dpp_f64(double identity, double v) {
    const uint64_t i = (uint64_t)__double_as_longlong(identity), x = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = dpp_u32<CTRL, ROWS>((uint32_t)i, (uint32_t)x);
    const uint32_t hi = dpp_u32<CTRL, ROWS>((uint32_t)(i >> 32), (uint32_t)(x >> 32));
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// max over the wave's 64 lanes (fmaxf: NaN lanes are ignored unless all are NaN)
__device__ __forceinline__ float wave_max_f32(float v) {
    v = fmaxf(v, dpp_f32<0xb1, 0xf>(v, v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f32<0x4e, 0xf>(v, v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_f32<0x114, 0xf>(v, v));  // row_shr 4
    v = fmaxf(v, dpp_f32<0x118, 0xf>(v, v));  // row_shr 8
    v = fmaxf(v, dpp_f32<0x142, 0xa>(v, v));  // row_bcast 15
    v = fmaxf(v, dpp_f32<0x143, 0xc>(v, v));  // row_bcast 31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// sum over the wave's 64 lanes in double, a fixed addition tree
__device__ __forceinline__ double wave_sum_f64(double v) {
    v += dpp_f64<0xb1, 0xf>(0.0, v);
    v += dpp_f64<0x4e, 0xf>(0.0, v);
    v += dpp_f64<0x114, 0xf>(0.0, v);
    v += dpp_f64<0x118, 0xf>(0.0, v);
    v += dpp_f64<0x142, 0xa>(0.0, v);
    v += dpp_f64<0x143, 0xc>(0.0, v);
    const uint64_t x = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), 63);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

}  // namespace hip
}  // namespace vla
