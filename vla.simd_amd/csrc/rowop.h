// rowop.h - the per-row ops that produce int8 GEMM inputs (identity,
// LayerNorm, RMSNorm, SiLU-gate), shared by the standalone row kernel
// (eltwise.hip rowq_kernel) and the skinny GEMM that builds its own
// activations (gemm_i8.hip), so both give the same floats and bytes.
//
// One wave owns a row held in registers: lane l has elements 4 l + 256 i,
// i < NV (zero past H). LayerNorm follows src/hal/common/norms.cpp:69-97 and
// RMSNorm :19-35 (statistics in double, inv rounded once to float, output
// formed in float); SiLU-gate is act_silu_gate (eltwise.cpp:29-64).
// Include it before any `#pragma clang fp contract` so every translation unit
// compiles these functions under the same contraction setting.
#pragma once

#include "act.h"
#include "quant_row.h"

namespace vla {
namespace hip {

// y <- the row xr[0, H) (zero past H). Rows are 16-byte aligned.
template <int NV>
__device__ __forceinline__ void rowop_load(float4 (&y)[NV], const float* xr, int H, int lane) {
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int k = 4 * lane + 256 * i;
        y[i] = k < H ? *reinterpret_cast<const float4*>(xr + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

// The row statistics of a norm (op 1: mean and inverse deviation; op 2: the
// inverse root mean square), from the row in registers. Split from the
// element-wise part so a wave can keep several rows' reductions in flight.
struct RowStat {
    double mean;
    float inv;
};

template <int OP, int NV>
__device__ __forceinline__ RowStat rowop_stat(const float4 (&y)[NV], float eps, int H, int lane) {
    RowStat st{0.0, 1.0f};
    if (OP == 1) {
        double s = 0.0;
#pragma unroll
        for (int i = 0; i < NV; i++)
            s += ((double)y[i].x + (double)y[i].y) + ((double)y[i].z + (double)y[i].w);
        const double mean = wave_sum_f64(s) / H;
        double v = 0.0;
#pragma unroll
        for (int i = 0; i < NV; i++)
            if (4 * lane + 256 * i < H) {
                const double d0 = (double)y[i].x - mean, d1 = (double)y[i].y - mean;
                const double d2 = (double)y[i].z - mean, d3 = (double)y[i].w - mean;
                v += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
            }
        st.mean = mean;
        st.inv = (float)(1.0 / sqrt(wave_sum_f64(v) / H + (double)eps));
    } else if (OP == 2) {
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const double d0 = y[i].x, d1 = y[i].y, d2 = y[i].z, d3 = y[i].w;
            ss += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
        }
        st.inv = (float)(1.0 / sqrt(wave_sum_f64(ss) / H + (double)eps));
    }
    return st;
}

// y <- op(y) given the row's statistics: op 0 identity, 1 LayerNorm (w, b or
// null), 2 RMSNorm (w), 3 silu_gate(y, ur). Weights and ur are 16-byte
// aligned; elements past H stay zero.
template <int OP, int NV>
__device__ __forceinline__ void rowop_finish(float4 (&y)[NV], RowStat st, const float* ur, const float* w,
                                             const float* b, int H, int lane) {
    if (OP == 1) {
        const double mean = st.mean;
        const float inv = st.inv;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int k = 4 * lane + 256 * i;
            if (k < H) {
                const float4 wv = *reinterpret_cast<const float4*>(w + k);
                float4 r;
                if (b) {
                    const float4 bv = *reinterpret_cast<const float4*>(b + k);
                    r.x = fmaf((float)((double)y[i].x - mean) * inv, wv.x, bv.x);
                    r.y = fmaf((float)((double)y[i].y - mean) * inv, wv.y, bv.y);
                    r.z = fmaf((float)((double)y[i].z - mean) * inv, wv.z, bv.z);
                    r.w = fmaf((float)((double)y[i].w - mean) * inv, wv.w, bv.w);
                } else {
                    r.x = (float)((double)y[i].x - mean) * inv * wv.x;
                    r.y = (float)((double)y[i].y - mean) * inv * wv.y;
                    r.z = (float)((double)y[i].z - mean) * inv * wv.z;
                    r.w = (float)((double)y[i].w - mean) * inv * wv.w;
                }
                y[i] = r;
            }
        }
    } else if (OP == 2) {
        const float inv = st.inv;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int k = 4 * lane + 256 * i;
            if (k < H) {
                const float4 wv = *reinterpret_cast<const float4*>(w + k);
                y[i] = make_float4(y[i].x * inv * wv.x, y[i].y * inv * wv.y, y[i].z * inv * wv.z,
                                   y[i].w * inv * wv.w);
            }
        }
    } else if (OP == 3) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int k = 4 * lane + 256 * i;
            if (k < H) {
                const float4 u = *reinterpret_cast<const float4*>(ur + k);
                y[i] = make_float4(act_silu_gate(y[i].x, u.x), act_silu_gate(y[i].y, u.y),
                                   act_silu_gate(y[i].z, u.z), act_silu_gate(y[i].w, u.w));
            }
        }
    }
}

template <int OP, int NV>
__device__ __forceinline__ void rowop_apply(float4 (&y)[NV], const float* xr, const float* ur,
                                            const float* w, const float* b, float eps, int H, int lane) {
    rowop_load<NV>(y, xr, H, lane);
    rowop_finish<OP, NV>(y, rowop_stat<OP, NV>(y, eps, H, lane), ur, w, b, H, lane);
}

// This lane's part of the row's max |y| (elements past H are zero).
template <int NV>
__device__ __forceinline__ float rowop_amax(const float4 (&y)[NV], int H, int lane) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++)
        if (4 * lane + 256 * i < H)
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(y[i].x), fabsf(y[i].y)), fmaxf(fabsf(y[i].z), fabsf(y[i].w))));
    return amax;
}

// The row's int8 scale (quant_ops.h:17-21) from its values in registers.
template <int NV>
__device__ __forceinline__ float rowop_scale(const float4 (&y)[NV], int H, int lane) {
    return row_scale(wave_max_f32(rowop_amax<NV>(y, H, lane)));
}

}  // namespace hip
}  // namespace vla
