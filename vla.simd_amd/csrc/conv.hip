// conv.hip - W8A8 2-D convolution on the int8 GEMM: conv2d_i8 of
// src/ops/conv_ops.h:31-35 (src/hal/common/conv.cpp:424-526).
//
// NHWC input x [H, Wd, Cin] fp32, weights [Cout][k][k][Cin] quantized per
// output channel over K = k*k*Cin, one activation scale for the whole input:
//   amax = max |x|; s = amax > 0 ? max(amax * clip / 127, FLT_MIN) : 1 with
//   clip = TCPU_I8_CLIP in (0, 1] (default 1), q = clamp(rne(x * (1/s)), +-127)
//   (quantize_tensor_i8, conv.cpp:448-465; quantize_span_i8, gemm_i8.cpp:177-206),
// and out[p][co] = fma((float)acc * ws[co], s, b[co]) where acc is output
// pixel p's patch -- taps [ky][kx][ci] at (oy*stride - pad + ky,
// ox*stride - pad + kx), zero outside the image (conv.cpp:117-176) -- dotted
// with channel co's weights: dense_linear_i8_pre over the im2col rows with
// every row scale s.
//
// Three launches on the caller's stream (two when the producer of x passes
// the block maxima of |x| it wrote, ConvArgs::in_part):
//   conv_absmax_kernel  per-block max |x| (float4 loads, wave + LDS reduce);
//   conv_im2col_kernel  every block first folds the block maxima into the
//                       scale (a few hundred floats; the same value in every
//                       block, no atomics), then its waves write im2col rows
//                       straight from fp32 x, 4-byte words at a time -- one
//                       float4 load when the 4 bytes are 4 channels of one
//                       tap -- and their row scales; rows are 64-byte padded,
//                       so the GEMM takes its aligned kernels;
//   launch_gemm_i8      the int8 GEMM with its fused epilogue.
// The im2col matrix is materialised: npix * round64(K) bytes (e.g. 11 MiB for
// a 480x640 ResNet stem), a few microseconds of HBM next to the GEMM.
#include "common.h"
#include "quant_row.h"

#include <cfloat>
#include <cstdlib>

#pragma clang fp contract(off)

namespace vla {
namespace hip {
namespace {

constexpr int kAbsmaxBlocks = 512;

__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max_f32(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    v = 0.0f;
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) v = fmaxf(v, red[w]);
    return v;
}

__global__ __launch_bounds__(256) void conv_absmax_kernel(const float* __restrict__ x, int64_t n,
                                                          float* __restrict__ part) {
    __shared__ float red[4];
    float m = 0.0f;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if ((reinterpret_cast<uintptr_t>(x) & 15) == 0) {
        const int64_t n4 = n / 4;
        for (int64_t i = t0; i < n4; i += stride) {
            const float4 v = reinterpret_cast<const float4*>(x)[i];
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
        for (int64_t i = n4 * 4 + t0; i < n; i += stride) m = fmaxf(m, fabsf(x[i]));
    } else {
        for (int64_t i = t0; i < n; i += stride) m = fmaxf(m, fabsf(x[i]));
    }
    m = block_max(m, red);
    if (threadIdx.x == 0) part[blockIdx.x] = m;
}

struct Im2colArgs {
    const float* x;
    int H, Wd, Cin, k, stride, pad, Wout;
    int npix, K, lda;
    const float* part;
    int nparts;
    float clip;
    int8_t* A;
    float* ascale;
};

// im2col work: groups of kIm2colRows consecutive output pixels x chunks of 64
// word columns. The groups are cut into 8 contiguous bands, one per XCD
// (block b runs on XCD b % 8), so each XCD's L2 holds only its band's input
// rows; inside a band the XCD's waves form rows of nchunk waves, and wave
// (row wr, chunk ch) takes the band's groups wr, wr + rows, ... of chunk ch.
constexpr int kIm2colRows = 8;
constexpr int kIm2colMaxBlocks = 2048;

// Each block folds the block maxima into the scale once. Each wave then
// decomposes its lanes' word columns (lane l: column 64 ch + l, 4 bytes of
// the patch -- one tap's 4 channels when VEC, else up to 4 taps' channels)
// into (ky, kx, ci) once, and for each of its pixel groups issues the loads
// of all kIm2colRows pixels before converting any and stores one word per
// pixel. Pixel coordinates advance incrementally: no integer division per
// word or per pixel.
template <bool VEC>
__global__ __launch_bounds__(256) void conv_im2col_kernel(Im2colArgs a) {
    __shared__ float red[4];
    float m = 0.0f;
    for (int i = threadIdx.x; i < a.nparts; i += blockDim.x) m = fmaxf(m, a.part[i]);
    const float amax = block_max(m, red);
    float s = 1.0f;
    if (amax > 0.0f) {
        const float t = amax * a.clip;
        s = t / 127.0f;
        s = s > FLT_MIN ? s : FLT_MIN;
    }
    const float inv = 1.0f / s;

    const float* __restrict__ x = a.x;
    const int lane = threadIdx.x & 63;
    const int wpr = a.lda / 4, nchunk = (wpr + 63) / 64;
    const int xcd = blockIdx.x & 7;
    const int lw = (blockIdx.x >> 3) * 4 + (threadIdx.x >> 6), rows = (gridDim.x >> 3) * 4 / nchunk;
    const int ch = lw % nchunk, wr = lw / nchunk;
    if (wr >= rows) return;
    const int cw = ch * 64 + lane, c = cw * 4;
    const bool col = cw < wpr;
    const int kc = a.k * a.Cin;
    int dy[4], dx[4], ci[4];
    bool live[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int kk = c + (VEC ? 0 : j);
        live[j] = col && c + j < a.K;
        const int r = kk % kc;
        dy[j] = kk / kc;
        dx[j] = r / a.Cin;
        ci[j] = r % a.Cin;
    }
    const int ngroup = (a.npix + kIm2colRows - 1) / kIm2colRows;
    const int g1 = (int)((int64_t)(xcd + 1) * ngroup / 8);
    for (int g = (int)((int64_t)xcd * ngroup / 8) + wr; g < g1; g += rows) {
        const int p0 = g * kIm2colRows;
        int oy = p0 / a.Wout, ox = p0 - oy * a.Wout;
        float v[kIm2colRows][4];
#pragma unroll
        for (int rr = 0; rr < kIm2colRows; rr++) {
            const int y0 = oy * a.stride - a.pad, x0 = ox * a.stride - a.pad;
            if (VEC) {
                const int iy = y0 + dy[0], ix = x0 + dx[0];
                float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
                if (live[0] && iy >= 0 && iy < a.H && ix >= 0 && ix < a.Wd)
                    f = *reinterpret_cast<const float4*>(x + (iy * a.Wd + ix) * a.Cin + ci[0]);
                v[rr][0] = f.x;
                v[rr][1] = f.y;
                v[rr][2] = f.z;
                v[rr][3] = f.w;
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int iy = y0 + dy[j], ix = x0 + dx[j];
                    v[rr][j] = live[j] && iy >= 0 && iy < a.H && ix >= 0 && ix < a.Wd
                                   ? x[(iy * a.Wd + ix) * a.Cin + ci[j]]
                                   : 0.0f;
                }
            }
            if (++ox == a.Wout) {
                ox = 0;
                oy++;
            }
        }
        if (!col) continue;
#pragma unroll
        for (int rr = 0; rr < kIm2colRows; rr++) {
            const int p = p0 + rr;
            if (p >= a.npix) break;
            reinterpret_cast<uint32_t*>(a.A + (size_t)p * a.lda)[cw] =
                q8x4(make_float4(v[rr][0], v[rr][1], v[rr][2], v[rr][3]), inv);
            if (cw == 0) a.ascale[p] = s;
        }
    }
}

float clip_from_env() {
    // TCPU_I8_CLIP as the reference reads it (src/hal/common/env.cpp:220-226):
    // a value in (0, 1], else 1
    static const float v = [] {
        const char* e = std::getenv("TCPU_I8_CLIP");
        const float f = e ? (float)std::atof(e) : 1.0f;
        return f > 0.0f && f <= 1.0f ? f : 1.0f;
    }();
    return v;
}

}  // namespace

ConvShape conv_shape(int H, int Wd, int Cin, int k, int stride, int pad, int Cout) {
    VLA_REQUIRE(H > 0 && Wd > 0 && Cin > 0 && Cout > 0 && k > 0 && stride > 0 && pad >= 0,
                "conv2d_i8: need positive H, Wd, Cin, Cout, k, stride and pad >= 0");
    // all extents in 64-bit before any of them is derived (a pad near 2^30
    // must not wrap H + 2 * pad)
    const int64_t hp = (int64_t)H + 2 * (int64_t)pad, wp = (int64_t)Wd + 2 * (int64_t)pad;
    VLA_REQUIRE(hp >= k && wp >= k, "conv2d_i8: kernel larger than the padded input");
    VLA_REQUIRE((int64_t)k * k * Cin <= kMaxI8K, "conv2d_i8: K = k*k*Cin exceeds INT_MAX/(255*127)");
    const int64_t ho = (hp - k) / stride + 1, wo = (wp - k) / stride + 1;
    VLA_REQUIRE(ho * wo < (1 << 30) && (int64_t)H * Wd * Cin < ((int64_t)1 << 31),
                "conv2d_i8: input or output too large");
    ConvShape c;
    c.Hout = (int)ho;
    c.Wout = (int)wo;
    c.K = k * k * Cin;
    VLA_REQUIRE((int64_t)c.Hout * c.Wout < (1 << 30) && (int64_t)H * Wd * Cin < ((int64_t)1 << 31),
                "conv2d_i8: input or output too large");
    c.npix = c.Hout * c.Wout;
    c.lda = (kpad4(c.K) + 63) & ~63;
    c.split = gemm_split_bytes(c.npix, Cout, c.K);
    c.work = (size_t)kAbsmaxBlocks * 4 + ((size_t)c.npix * 4 + 255) / 256 * 256 +
             ((size_t)c.npix * c.lda + 255) / 256 * 256 + c.split;
    return c;
}

void launch_conv2d_i8(const ConvArgs& a, hipStream_t st) {
    const ConvShape c = conv_shape(a.H, a.Wd, a.Cin, a.k, a.stride, a.pad, a.Cout);
    VLA_REQUIRE(a.x && a.out && a.Wq && a.wscale && a.work, "conv2d_i8: null buffer");
    VLA_REQUIRE(a.ldw >= kpad4(c.K) && a.ldw % 4 == 0, "conv2d_i8: bad weight rows");
    VLA_REQUIRE(a.work_bytes >= c.work, "conv2d_i8: workspace too small (vla_conv2d_i8_workspace_bytes)");
    VLA_REQUIRE((reinterpret_cast<uintptr_t>(a.work) & 255) == 0, "conv2d_i8: workspace must be 256-byte aligned");
    char* w = static_cast<char*>(a.work);
    // [block maxima: 512 floats][row scales: npix floats][im2col rows][split-K sums],
    // each 256-byte rounded
    float* part = reinterpret_cast<float*>(w);
    float* ascale = reinterpret_cast<float*>(w + (size_t)kAbsmaxBlocks * 4);
    int8_t* A = reinterpret_cast<int8_t*>(w + (size_t)kAbsmaxBlocks * 4 + ((size_t)c.npix * 4 + 255) / 256 * 256);

    int blocks;
    const float* maxima = part;
    if (a.in_part) {
        // the producer of x wrote its block maxima: no pass over x here
        VLA_REQUIRE(a.in_nparts > 0 && a.in_nparts <= 4096, "conv2d_i8: 1..4096 producer block maxima");
        maxima = a.in_part;
        blocks = a.in_nparts;
    } else {
        const int64_t n = (int64_t)a.H * a.Wd * a.Cin;
        blocks = (int)((n + 4 * 256 * 4 - 1) / (4 * 256 * 4));
        blocks = blocks < 1 ? 1 : (blocks > kAbsmaxBlocks ? kAbsmaxBlocks : blocks);
        conv_absmax_kernel<<<blocks, 256, 0, st>>>(a.x, n, part);
        VLA_LAUNCH_CHECK();
    }

    Im2colArgs g{a.x, a.H, a.Wd, a.Cin, a.k, a.stride, a.pad, c.Wout, c.npix, c.K, c.lda, maxima, blocks,
                 a.clip > 0.0f ? a.clip : clip_from_env(), A, ascale};
    // enough waves for every (group, chunk), at most kIm2colMaxBlocks blocks,
    // a multiple of 8 blocks, and at least one row of nchunk waves per XCD
    const int nchunk = (c.lda / 4 + 63) / 64;
    const int64_t tasks = (int64_t)((c.npix + kIm2colRows - 1) / kIm2colRows) * nchunk;
    int per_xcd = (int)((tasks + 31) / 32 < kIm2colMaxBlocks / 8 ? (tasks + 31) / 32 : kIm2colMaxBlocks / 8);
    per_xcd = per_xcd * 4 < nchunk ? (nchunk + 3) / 4 : per_xcd;
    const int gb = per_xcd * 8;
    if (a.Cin % 4 == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0)
        conv_im2col_kernel<true><<<gb, 256, 0, st>>>(g);
    else
        conv_im2col_kernel<false><<<gb, 256, 0, st>>>(g);
    VLA_LAUNCH_CHECK();

    GemmArgs m{};
    m.A = A;
    m.lda = c.lda;
    m.B = a.Wq;
    m.ldb = a.ldw;
    m.ascale = ascale;
    m.wscale = a.wscale;
    m.bias = a.bias;
    m.out = a.out;
    m.ldo = a.Cout;
    m.M = c.npix;
    m.N = a.Cout;
    m.K = c.K;
    if (c.split) {
        m.split_ws = reinterpret_cast<int32_t*>(w + c.work - c.split);
        m.split_bytes = c.split;
    }
    launch_gemm_i8(m, st);
}

}  // namespace hip
}  // namespace vla
