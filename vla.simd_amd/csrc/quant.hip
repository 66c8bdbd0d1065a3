// quant.hip - per-row dynamic int8 quantization on gfx950.
//
// Numeric contract (src/ops/quant_ops.h:17-21, src/hal/common/gemm_i8.cpp:49-54,
// 132-171, 209-244): per row, amax = max_k |x|; s = amax > 0 ?
// max(amax/127, FLT_MIN) : 1; inv = 1/s; q = clamp(rne(x*inv), -127, 127);
// columns [K, ldq) are zero. Every step is exact or a single IEEE-rounded
// operation (max is exact; the two divisions are correctly rounded - hipcc
// emits the v_div_scale/v_div_fmas/v_div_fixup sequence for '/', never v_rcp
// alone; the product is one v_mul_f32; v_rndne_f32 is round-half-even), so the
// result does not depend on the order lanes visit the row and is bit-identical
// to the reference's scalar and AVX2 quantizers. fp32 denormals are preserved
// (no -fgpu-flush-denormals-to-zero), which the FLT_MIN floor relies on.
//
// Layout: one wave64 per row, four rows per 256-thread block. A lane reads
// float4 runs (coalesced 1 KiB per wave instruction). Rows up to 4096 floats
// stay in registers between the max and the quantize pass, so each element is
// read once; longer rows are read twice, the second time from L1/L2.

#include "common.h"
#include "quant_row.h"

#include <cstdlib>

#pragma clang fp contract(off)

namespace vla {
namespace hip {
namespace {

// VEC: rows are 16-byte aligned and K % 4 == 0, so float4 loads cover the row.
template <bool VEC>
__global__ __launch_bounds__(256) void quantize_rows_kernel(const float* __restrict__ x, int ldx,
                                                            int8_t* __restrict__ xq, int ldq,
                                                            float* __restrict__ scale, int rows,
                                                            int K) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;  // wave-uniform
    const float* xr = x + (size_t)row * ldx;

    float amax = 0.0f;
    if (VEC) {
        for (int k = lane * 4; k < K; k += 256) {
            const float4 v = *reinterpret_cast<const float4*>(xr + k);
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
    } else {
        for (int k = lane; k < K; k += 64) amax = fmaxf(amax, fabsf(xr[k]));
    }
    amax = wave_max_f32(amax);
    const float s = row_scale(amax);
    const float inv = 1.0f / s;
    if (lane == 0) scale[row] = s;

    // ldq % 4 == 0 and the row base is 4-byte aligned (checked by the launcher),
    // so each lane writes whole 32-bit words covering [0, ldq).
    int8_t* qr = xq + (size_t)row * ldq;
    for (int k = lane * 4; k < ldq; k += 256) {
        uint32_t word = 0;
        if (VEC && k + 4 <= K) {
            const float4 v = *reinterpret_cast<const float4*>(xr + k);
            word = q8x4(v, inv);
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int kk = k + j;
                const int q = kk < K ? q8(xr[kk], inv) : 0;
                word |= (uint32_t)(q & 0xff) << (8 * j);
            }
        }
        *reinterpret_cast<uint32_t*>(qr + k) = word;
    }
}

// Rows of at most 256 * NV floats, 16-byte aligned, K % 4 == 0: the row is
// held in registers (NV float4 per lane), so it is read once, from HBM.
template <int NV>
__global__ __launch_bounds__(256) void quantize_rows_reg(const float* __restrict__ x, int ldx,
                                                         int8_t* __restrict__ xq, int ldq,
                                                         float* __restrict__ scale, int rows, int K) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;  // wave-uniform
    const float* xr = x + (size_t)row * ldx;
    float4 v[NV];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int k = 4 * lane + 256 * i;
        v[i] = k < K ? *reinterpret_cast<const float4*>(xr + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    }
    amax = wave_max_f32(amax);
    const float s = row_scale(amax);
    const float inv = 1.0f / s;
    if (lane == 0) scale[row] = s;
    int8_t* qr = xq + (size_t)row * ldq;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int k = 4 * lane + 256 * i;
        if (k < K) *reinterpret_cast<uint32_t*>(qr + k) = q8x4(v[i], inv);
    }
    // the zero pad [K, ldq) (whole words: K % 4 == 0 and ldq % 4 == 0)
    for (int k = K + 4 * lane; k < ldq; k += 256) *reinterpret_cast<uint32_t*>(qr + k) = 0u;
}

// Long rows (K >= 2048, 16-byte aligned, K % 4 == 0), row-major: a block per
// row, NV float4 per thread (16 VGPRs of row data at K = 4096 instead of the
// wave-per-row kernel's 64), so eight rows' loads are in flight per CU at once
// and a grid of thousands of rows runs in full rounds of resident blocks. The
// block max goes through LDS; the max is exact in any order, so the bytes and
// the scale are the wave-per-row kernel's.
template <int NV>
__global__ __launch_bounds__(256) void quantize_rows_wide(const float* __restrict__ x, int ldx,
                                                          int8_t* __restrict__ xq, int ldq,
                                                          float* __restrict__ scale, int K) {
    __shared__ float red[4];
    const int t = threadIdx.x, row = blockIdx.x;
    const float* xr = x + (size_t)row * ldx;
    float4 v[NV];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int k = 4 * (t + 256 * i);
        v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (k < K) {
            v[i] = *reinterpret_cast<const float4*>(xr + k);
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
        }
    }
    amax = wave_max_f32(amax);
    if ((t & 63) == 0) red[t >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s = row_scale(amax);
    const float inv = 1.0f / s;
    if (t == 0) scale[row] = s;
    int8_t* qr = xq + (size_t)row * ldq;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int k = 4 * (t + 256 * i);
        if (k < K) *reinterpret_cast<uint32_t*>(qr + k) = q8x4(v[i], inv);
    }
    // the zero pad [K, ldq) (whole words: K % 4 == 0 and ldq % 4 == 0)
    for (int k = K + 4 * t; k < ldq; k += 1024) *reinterpret_cast<uint32_t*>(qr + k) = 0u;
}

// The same quantization written in the panel layout (common.h): word (m, k)
// of a row lands at (k / 64) * mp * 64 + m * 64 + k % 64; bytes [K, K64) of
// the row are zero. Rows are few (<= 128), so the row is simply read twice.
template <bool VEC>
__global__ __launch_bounds__(256) void quantize_rows_panel_kernel(const float* __restrict__ x, int ldx,
                                                                  int8_t* __restrict__ xq, int mp,
                                                                  float* __restrict__ scale, int rows,
                                                                  int K) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;  // wave-uniform
    const float* xr = x + (size_t)row * ldx;
    float amax = 0.0f;
    if (VEC) {
        for (int k = lane * 4; k < K; k += 256) {
            const float4 v = *reinterpret_cast<const float4*>(xr + k);
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
    } else {
        for (int k = lane; k < K; k += 64) amax = fmaxf(amax, fabsf(xr[k]));
    }
    amax = wave_max_f32(amax);
    const float s = row_scale(amax);
    const float inv = 1.0f / s;
    if (lane == 0) scale[row] = s;
    const int k64 = (K + 63) & ~63;
    int8_t* base = xq + (size_t)row * 64;
    for (int k = lane * 4; k < k64; k += 256) {
        uint32_t word = 0;
        if (VEC && k + 4 <= K) {
            word = q8x4(*reinterpret_cast<const float4*>(xr + k), inv);
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int kk = k + j;
                const int q = kk < K ? q8(xr[kk], inv) : 0;
                word |= (uint32_t)(q & 0xff) << (8 * j);
            }
        }
        *reinterpret_cast<uint32_t*>(base + (size_t)(k >> 6) * mp * 64 + (k & 63)) = word;
    }
}

// Rows of at most 256 * NV floats (VEC) in the panel layout: the row in
// registers, every load in flight at once (the loop form above waits for each
// load before issuing the next); same bytes and scale.
template <int NV>
__global__ __launch_bounds__(256) void quantize_rows_panel_reg(const float* __restrict__ x, int ldx,
                                                               int8_t* __restrict__ xq, int mp,
                                                               float* __restrict__ scale, int rows, int K) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;  // wave-uniform
    const float* xr = x + (size_t)row * ldx;
    float4 v[NV];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int k = 4 * lane + 256 * i;
        v[i] = k < K ? *reinterpret_cast<const float4*>(xr + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    }
    amax = wave_max_f32(amax);
    const float s = row_scale(amax);
    const float inv = 1.0f / s;
    if (lane == 0) scale[row] = s;
    const int k64 = (K + 63) & ~63;
    int8_t* base = xq + (size_t)row * 64;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int k = 4 * lane + 256 * i;
        if (k < k64)  // K % 4 == 0: a float4 is wholly inside [0, K) or wholly padding
            *reinterpret_cast<uint32_t*>(base + (size_t)(k >> 6) * mp * 64 + (k & 63)) = k < K ? q8x4(v[i], inv) : 0u;
    }
}

// Long rows (K >= 2048) in the panel layout: a block per row, the row held in
// registers (NV float4 per thread), so every load is in flight at once and
// the row is read once; the block max goes through LDS. Same bytes and scale
// as the wave-per-row kernel (the max is exact in any order).
template <int NV, int NT = 256>
__global__ __launch_bounds__(NT) void quantize_rows_panel_wide(const float* __restrict__ x, int ldx,
                                                               int8_t* __restrict__ xq, int mp,
                                                               float* __restrict__ scale, int K) {
    __shared__ float red[NT / 64];
    const int t = threadIdx.x, row = blockIdx.x;
    const float* xr = x + (size_t)row * ldx;
    float4 v[NV];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int k = 4 * (t + NT * i);
        v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (k < K) {
            v[i] = *reinterpret_cast<const float4*>(xr + k);
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
        }
    }
    amax = wave_max_f32(amax);
    if ((t & 63) == 0) red[t >> 6] = amax;
    __syncthreads();
    amax = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; w++) amax = fmaxf(amax, red[w]);
    const float s = row_scale(amax);
    const float inv = 1.0f / s;
    if (t == 0) scale[row] = s;
    const int k64 = (K + 63) & ~63;
    int8_t* base = xq + (size_t)row * 64;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int k = 4 * (t + NT * i);
        if (k < k64)  // K % 4 == 0: a float4 is wholly inside [0, K) or wholly padding
            *reinterpret_cast<uint32_t*>(base + (size_t)(k >> 6) * mp * 64 + (k & 63)) = k < K ? q8x4(v[i], inv) : 0u;
    }
}

// quantize_span_i8 (src/ops/quant_ops.h:78-80, gemm_i8.cpp:177-207): one
// shared inverse scale, q = clamp(rne(x * inv), +-127), the same q8 as the row
// quantizers. VEC: 4 elements per thread (x 16-byte and q 4-byte aligned).
template <bool VEC>
__global__ __launch_bounds__(256) void quantize_span_kernel(const float* __restrict__ x, int8_t* __restrict__ q,
                                                            int64_t n, float inv) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (VEC) {
        for (; 4 * i + 3 < n; i += stride)
            reinterpret_cast<uint32_t*>(q)[i] = q8x4(reinterpret_cast<const float4*>(x)[i], inv);
        // the tail (n % 4 elements) by the first threads
        const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
        const int64_t e = (n & ~(int64_t)3) + t;
        if (t < 4 && e < n) q[e] = (int8_t)q8(x[e], inv);
    } else {
        for (; i < n; i += stride) q[i] = (int8_t)q8(x[i], inv);
    }
}

}  // namespace

void launch_quantize_span(const float* x, int8_t* q, int64_t n, float inv, hipStream_t st) {
    VLA_REQUIRE(n >= 0, "quantize_span: n must be >= 0");
    VLA_REQUIRE(n == 0 || (x && q), "quantize_span: null buffer");
    if (n == 0) return;
    const bool vec = aligned(x, 16) && aligned(q, 4);
    const int64_t work = vec ? (n + 3) / 4 : n;
    const int blocks = (int)((work + 255) / 256 < 4096 ? (work + 255) / 256 : 4096);
    if (vec) quantize_span_kernel<true><<<blocks, 256, 0, st>>>(x, q, n, inv);
    else quantize_span_kernel<false><<<blocks, 256, 0, st>>>(x, q, n, inv);
    VLA_LAUNCH_CHECK();
}

void launch_quantize_rows_panel(const float* x, int ldx, int8_t* xq, float* scale, int rows, int K,
                                hipStream_t st, bool taps) {
    VLA_REQUIRE(rows >= 0 && rows <= kPanelMaxRows && K > 0,
                "quantize (panel): rows must be in [0, 128] and K > 0");
    VLA_REQUIRE(ldx >= K || (taps && ldx > 0), "quantize (panel): ldx < K");
    VLA_REQUIRE(aligned(xq, 4), "quantize (panel): xq must be 4-byte aligned");
    if (rows == 0) return;
    const int mp = panel_rows(rows);
    const dim3 grid((rows + 3) / 4), block(256);
    const bool vec = K % 4 == 0 && ldx % 4 == 0 && aligned(x, 16);
    const int nv = ((K + 63) / 64 * 64 + 1023) / 1024;  // float4 per thread over [0, K64), block per row
    const int nvw = ((K + 63) / 64 * 64 + 255) / 256;   // float4 per lane over [0, K64), wave per row
    const int nv4 = (nv + 3) / 4;  // float4 per thread at 1024 threads per row
    if (vec && K > 8192 && rows <= 32 && nv4 <= 8) {
        // few long rows (a 1-D convolution's taps, K = 5 C): 1024 threads per
        // row, so each holds at most 8 float4 and the row's loads finish sooner
        if (nv4 <= 1) quantize_rows_panel_wide<1, 1024><<<rows, 1024, 0, st>>>(x, ldx, xq, mp, scale, K);
        else if (nv4 <= 2) quantize_rows_panel_wide<2, 1024><<<rows, 1024, 0, st>>>(x, ldx, xq, mp, scale, K);
        else if (nv4 <= 4) quantize_rows_panel_wide<4, 1024><<<rows, 1024, 0, st>>>(x, ldx, xq, mp, scale, K);
        else quantize_rows_panel_wide<8, 1024><<<rows, 1024, 0, st>>>(x, ldx, xq, mp, scale, K);
    } else if (vec && K >= 2048 && nv <= 16) {
        // one block per row: 64 x 12288 (SigLIP's projection input) 25.9 -> 6.6 us
        if (nv <= 4) quantize_rows_panel_wide<4><<<rows, 256, 0, st>>>(x, ldx, xq, mp, scale, K);
        else if (nv <= 8) quantize_rows_panel_wide<8><<<rows, 256, 0, st>>>(x, ldx, xq, mp, scale, K);
        else if (nv <= 12) quantize_rows_panel_wide<12><<<rows, 256, 0, st>>>(x, ldx, xq, mp, scale, K);
        else quantize_rows_panel_wide<16><<<rows, 256, 0, st>>>(x, ldx, xq, mp, scale, K);
    } else if (vec && nvw <= 8) {
        if (nvw <= 1) quantize_rows_panel_reg<1><<<grid, block, 0, st>>>(x, ldx, xq, mp, scale, rows, K);
        else if (nvw <= 2) quantize_rows_panel_reg<2><<<grid, block, 0, st>>>(x, ldx, xq, mp, scale, rows, K);
        else if (nvw <= 4) quantize_rows_panel_reg<4><<<grid, block, 0, st>>>(x, ldx, xq, mp, scale, rows, K);
        else quantize_rows_panel_reg<8><<<grid, block, 0, st>>>(x, ldx, xq, mp, scale, rows, K);
    } else if (vec)
        quantize_rows_panel_kernel<true><<<grid, block, 0, st>>>(x, ldx, xq, mp, scale, rows, K);
    else
        quantize_rows_panel_kernel<false><<<grid, block, 0, st>>>(x, ldx, xq, mp, scale, rows, K);
    VLA_LAUNCH_CHECK();
}

// Rows of at least this many floats take the block-per-row kernel;
// VLA_HIP_QUANT_WIDE_K overrides it per call (A/B runs: a value above 4096
// keeps every row on the wave-per-row kernels; the bytes never change).
static int wide_min_k() {
    const char* e = std::getenv("VLA_HIP_QUANT_WIDE_K");
    const int v = e ? std::atoi(e) : 0;
    return v > 0 ? v : 2048;
}

void launch_quantize_rows(const float* x, int ldx, int8_t* xq, int ldq, float* scale, int rows,
                          int K, hipStream_t st, bool taps) {
    VLA_REQUIRE(rows >= 0 && K > 0, "quantize: rows must be >= 0 and K > 0");
    VLA_REQUIRE(ldx >= K || (taps && ldx > 0), "quantize: ldx < K");
    VLA_REQUIRE(ldq >= kpad4(K) && ldq % 4 == 0, "quantize: ldq must be >= i8_kpad(K) and a multiple of 4");
    VLA_REQUIRE(aligned(xq, 4), "quantize: xq must be 4-byte aligned");
    if (rows == 0) return;
    const bool vec = K % 4 == 0 && ldx % 4 == 0 && aligned(x, 16);
    const dim3 grid((rows + 3) / 4), block(256);
    if (vec && K >= wide_min_k() && K <= 4 * 1024) {
        const int nv = (K + 1023) / 1024;
        if (nv <= 2) quantize_rows_wide<2><<<rows, block, 0, st>>>(x, ldx, xq, ldq, scale, K);
        else if (nv <= 3) quantize_rows_wide<3><<<rows, block, 0, st>>>(x, ldx, xq, ldq, scale, K);
        else quantize_rows_wide<4><<<rows, block, 0, st>>>(x, ldx, xq, ldq, scale, K);
    } else if (vec && K <= 16 * 256) {
        const int nv = (K + 255) / 256;
        if (nv <= 1) quantize_rows_reg<1><<<grid, block, 0, st>>>(x, ldx, xq, ldq, scale, rows, K);
        else if (nv <= 2) quantize_rows_reg<2><<<grid, block, 0, st>>>(x, ldx, xq, ldq, scale, rows, K);
        else if (nv <= 4) quantize_rows_reg<4><<<grid, block, 0, st>>>(x, ldx, xq, ldq, scale, rows, K);
        else if (nv <= 8) quantize_rows_reg<8><<<grid, block, 0, st>>>(x, ldx, xq, ldq, scale, rows, K);
        else quantize_rows_reg<16><<<grid, block, 0, st>>>(x, ldx, xq, ldq, scale, rows, K);
    } else if (vec)
        quantize_rows_kernel<true><<<grid, block, 0, st>>>(x, ldx, xq, ldq, scale, rows, K);
    else
        quantize_rows_kernel<false><<<grid, block, 0, st>>>(x, ldx, xq, ldq, scale, rows, K);
    VLA_LAUNCH_CHECK();
}

}  // namespace hip
}  // namespace vla
