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

// The op's per-element operands at this lane's elements: op 1 w (p) and b
// (q, when given), op 2 w (p), op 3 the up row ur (p); zero past H. Loaded
// right after the row, so no load waits behind the row's reduction.
template <int OP, int NV>
struct RowPar {
    float4 p[(OP >= 1 && OP <= 3) ? NV : 1], q[OP == 1 ? NV : 1];
};

template <int OP, int NV>
__device__ __forceinline__ void rowop_par(RowPar<OP, NV>& r, const float* ur, const float* w, const float* b, int H,
                                          int lane) {
    if constexpr (OP >= 1 && OP <= 3) {
        const float* src = OP == 3 ? ur : w;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int k = 4 * lane + 256 * i;
            r.p[i] = k < H ? *reinterpret_cast<const float4*>(src + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    if constexpr (OP == 1) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int k = 4 * lane + 256 * i;
            r.q[i] = b && k < H ? *reinterpret_cast<const float4*>(b + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
}

// y <- op(y) given the row's statistics and operands: op 0 identity, 1
// LayerNorm (w, b or none), 2 RMSNorm (w), 3 silu_gate(y, ur). Elements past
// H stay zero.
template <int OP, int NV>
__device__ __forceinline__ void rowop_finish_par(float4 (&y)[NV], RowStat st, const RowPar<OP, NV>& r, bool has_b,
                                                 int H, int lane) {
    if constexpr (OP == 1) {
        const double mean = st.mean;
        const float inv = st.inv;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int k = 4 * lane + 256 * i;
            if (k < H) {
                const float4 wv = r.p[i];
                float4 o;
                if (has_b) {
                    const float4 bv = r.q[i];
                    o.x = fmaf((float)((double)y[i].x - mean) * inv, wv.x, bv.x);
                    o.y = fmaf((float)((double)y[i].y - mean) * inv, wv.y, bv.y);
                    o.z = fmaf((float)((double)y[i].z - mean) * inv, wv.z, bv.z);
                    o.w = fmaf((float)((double)y[i].w - mean) * inv, wv.w, bv.w);
                } else {
                    o.x = (float)((double)y[i].x - mean) * inv * wv.x;
                    o.y = (float)((double)y[i].y - mean) * inv * wv.y;
                    o.z = (float)((double)y[i].z - mean) * inv * wv.z;
                    o.w = (float)((double)y[i].w - mean) * inv * wv.w;
                }
                y[i] = o;
            }
        }
    } else if constexpr (OP == 2) {
        const float inv = st.inv;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int k = 4 * lane + 256 * i;
            if (k < H) {
                const float4 wv = r.p[i];
                y[i] = make_float4(y[i].x * inv * wv.x, y[i].y * inv * wv.y, y[i].z * inv * wv.z,
                                   y[i].w * inv * wv.w);
            }
        }
    } else if constexpr (OP == 3) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int k = 4 * lane + 256 * i;
            if (k < H) {
                const float4 u = r.p[i];
                y[i] = make_float4(act_silu_gate(y[i].x, u.x), act_silu_gate(y[i].y, u.y),
                                   act_silu_gate(y[i].z, u.z), act_silu_gate(y[i].w, u.w));
            }
        }
    }
}

// rowop_finish_par with the operands loaded here (weights and ur 16-byte
// aligned).
template <int OP, int NV>
__device__ __forceinline__ void rowop_finish(float4 (&y)[NV], RowStat st, const float* ur, const float* w,
                                             const float* b, int H, int lane) {
    RowPar<OP, NV> r;
    rowop_par<OP, NV>(r, ur, w, b, H, lane);
    rowop_finish_par<OP, NV>(y, st, r, b != nullptr, H, lane);
}

template <int OP, int NV>
__device__ __forceinline__ void rowop_apply(float4 (&y)[NV], const float* xr, const float* ur,
                                            const float* w, const float* b, float eps, int H, int lane) {
    rowop_load<NV>(y, xr, H, lane);
    RowPar<OP, NV> r;
    rowop_par<OP, NV>(r, ur, w, b, H, lane);
    rowop_finish_par<OP, NV>(y, rowop_stat<OP, NV>(y, eps, H, lane), r, b != nullptr, H, lane);
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
