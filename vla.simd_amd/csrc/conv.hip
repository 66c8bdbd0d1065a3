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
// Input channels a multiple of 64 take an implicit GEMM where it measured
// faster: 1x1 convolutions, and k x k ones with at least 256 output tiles
// (MI355X, per call with the absmax pass: 120x160x64->64 3x3 19.3 -> 14.5 us,
// the 1x1 stride-2 downsamples 10.7 / 10.5 / 10.1 -> 9.7 / 9.3 / 9.8 us; with
// 40-150 tiles each block walks up to 72 K steps alone and the im2col rows
// + LDS-DMA GEMM win: 15x20x512 3x3 20.1 us against 33.3; a form whose 4
// waves each took every fourth K step of the whole tile was no faster, 24 us
// for its kernel alone: with about one block per CU and one slab of loads in
// flight, each step waits a memory latency, which the LDS-DMA GEMM's 3-4
// stages hide).
// VLA_HIP_CONV_IMPLICIT=0 turns it off (read per call):
//   conv_quant_kernel   the whole input quantized once to int8 NHWC (the
//                       scale folded from the block maxima in every block);
//   conv_i8_implicit    64 x 64 output tiles whose A slabs are gathered
//                       straight from that map: 64 channels of one tap per
//                       K step (zeros outside the image), double buffered
//                       through LDS, the same epilogue as the GEMM.
// Integer sums are exact in any order and the epilogue is the same one, so
// the outputs are bit-identical to the im2col path's.
//
// Otherwise three launches on the caller's stream (two when the producer of
// x passes the block maxima of |x| it wrote, ConvArgs::in_part):
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
#include "act.h"
#include "common.h"
#include "quant_row.h"

#include <cfloat>
#include <cstdlib>
#include <cstring>

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

// This thread's max over the block maxima part[0, nparts): float4 loads
// (16-byte aligned part), four issued before the first is used, so up to
// 4096 maxima cost one load latency per 256-thread block, not one per float.
__device__ __forceinline__ float parts_max(const float* __restrict__ part, int nparts) {
    float m = 0.0f;
    const int t = threadIdx.x, nt = blockDim.x;
    int done = 0;
    if ((reinterpret_cast<uintptr_t>(part) & 15) == 0) {
        const int n4 = nparts >> 2;
        const float4* p4 = reinterpret_cast<const float4*>(part);
        for (int b = 0; b < n4; b += 4 * nt) {
            float4 v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int i = b + j * nt + t;
                v[j] = i < n4 ? p4[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) m = fmaxf(fmaxf(m, fmaxf(v[j].x, v[j].y)), fmaxf(v[j].z, v[j].w));
        }
        done = n4 << 2;
    }
    for (int i = done + t; i < nparts; i += nt) m = fmaxf(m, part[i]);
    return m;
}

__global__ __launch_bounds__(256) void conv_absmax_kernel(const float* __restrict__ x, int64_t n,
                                                          float* __restrict__ part) {
    __shared__ float red[4];
    float m = 0.0f;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if ((reinterpret_cast<uintptr_t>(x) & 15) == 0) {
        const int64_t n4 = n / 4;
        const float4* x4 = reinterpret_cast<const float4*>(x);
        auto amax4 = [](float4 v) { return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))); };
        int64_t i = t0;
        // four loads in flight per thread (max is order-free: the same value)
        for (; i + 3 * stride < n4; i += 4 * stride) {
            const float4 a = x4[i], b = x4[i + stride], c = x4[i + 2 * stride], d = x4[i + 3 * stride];
            m = fmaxf(m, fmaxf(fmaxf(amax4(a), amax4(b)), fmaxf(amax4(c), amax4(d))));
        }
        for (; i < n4; i += stride) m = fmaxf(m, amax4(x4[i]));
        for (int64_t j = n4 * 4 + t0; j < n; j += stride) m = fmaxf(m, fabsf(x[j]));
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
    const float amax = block_max(parts_max(a.part, a.nparts), red);
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

// The per-tensor scale from the block maxima (every block folds them the
// same way, no atomics): s = amax > 0 ? max(amax * clip / 127, FLT_MIN) : 1.
__device__ __forceinline__ float fold_scale(const float* part, int nparts, float clip, float* red) {
    const float amax = block_max(parts_max(part, nparts), red);
    float s = 1.0f;
    if (amax > 0.0f) {
        const float t = amax * clip;
        s = t / 127.0f;
        s = s > FLT_MIN ? s : FLT_MIN;
    }
    return s;
}

// x [n4 float4] -> int8 NHWC q (quantize_tensor_i8, conv.cpp:448-465); the
// scale to s_out[0, nrows) (the GEMM's row scales)
__global__ __launch_bounds__(256) void conv_quant_kernel(const float4* __restrict__ x, int64_t n4,
                                                         uint32_t* __restrict__ q, const float* __restrict__ part,
                                                         int nparts, float clip, float* __restrict__ s_out,
                                                         int nrows) {
    __shared__ float red[4];
    const float s = fold_scale(part, nparts, clip, red);
    const float inv = 1.0f / s;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < nrows; i += gridDim.x * blockDim.x) s_out[i] = s;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x)
        q[i] = q8x4(x[i], inv);
}

// The trunk's max pool (-inf padding) + ReLU, the separate pass's
// expressions (a window max by v > o ? v : o, then relu_gt), whose output also
// goes out as the next conv's int8 map word q[e] with the scale folded from
// the maxima of max(0, x) the stem wrote: the same maxima as the pooled
// map's when every input pixel lies in some window. The scale to
// s_out[0, nrows) (the GEMM's row scales).
__global__ __launch_bounds__(256) void conv_pool_quant4_kernel(float4* __restrict__ out, const float4* __restrict__ x,
                                                               int H, int Wd, int C4, int k, int stride, int pad,
                                                               int Wout, int total4, const float* __restrict__ part,
                                                               int nparts, float clip, uint32_t* __restrict__ q,
                                                               float* __restrict__ s_out, int nrows) {
    __shared__ float red[4];
    const float s = fold_scale(part, nparts, clip, red);
    const float inv = 1.0f / s;
    for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < nrows; r += gridDim.x * blockDim.x) s_out[r] = s;
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < total4; e += gridDim.x * blockDim.x) {
        const int c4 = e % C4, p = e / C4;
        const int oy = p / Wout, ox = p - oy * Wout;
        float4 o = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        for (int ky = 0; ky < k; ky++) {
            const int iy = oy * stride - pad + ky;
            if (iy < 0 || iy >= H) continue;
            for (int kx = 0; kx < k; kx++) {
                const int ix = ox * stride - pad + kx;
                if (ix < 0 || ix >= Wd) continue;
                const float4 v = x[(iy * Wd + ix) * C4 + c4];
                o.x = v.x > o.x ? v.x : o.x;
                o.y = v.y > o.y ? v.y : o.y;
                o.z = v.z > o.z ? v.z : o.z;
                o.w = v.w > o.w ? v.w : o.w;
            }
        }
        const float4 r = make_float4(relu_gt(o.x), relu_gt(o.y), relu_gt(o.z), relu_gt(o.w));
        out[e] = r;
        q[e] = q8x4(r, inv);
    }
}

typedef int v4i __attribute__((ext_vector_type(4)));

struct ImplicitArgs {
    const int8_t* xq;  // int8 NHWC [H, Wd, Cin], Cin % 64 == 0
    int H, Wd, Cin, k, stride, pad, Wout, npix;
    const int8_t* W;   // [N][ldw], K = k * k * Cin in [ky][kx][ci] order
    int ldw;
    const float* wscale;
    const float* bias;
    const float* s;    // the activation scale (device)
    float* out;        // [npix, N]
    int N, K;
    // the trunk's fused epilogue: act 1 = ReLU, or resid [npix, N] added
    // before relu_gt; omax: each block's max |out| at [block]
    int act;
    const float* resid;
    float* omax;
};

// 64 x 64 output tile per block, 4 waves in a 2 x 2 grid (32 x 32 each: 2 x 2
// MFMA fragments). K step = 64 bytes = 64 channels of one tap (ky, kx): each
// thread loads one 16-byte chunk of one pixel's row for A and one of one
// output channel's weights for B; LDS rows of 64 + 16 bytes. The weight
// fragment goes first, so lane l holds output row l % 16 and the four
// consecutive channels 4 (l / 16) .. + 3, stored as one float4.
__global__ __launch_bounds__(256) void conv_i8_implicit(ImplicitArgs a) {
    constexpr int BM = 64, BN = 64, BK = 64, SP = BK + 16;
    __shared__ __attribute__((aligned(16))) int8_t sm[2][(BM + BN) * SP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int r = tid >> 2, q = (tid & 3) * 16;  // this thread's row of A and of B, its 16-byte chunk
    const int m = m0 + r < a.npix ? m0 + r : a.npix - 1;
    const int oy = m / a.Wout, ox = m - oy * a.Wout;
    const int iy0 = oy * a.stride - a.pad, ix0 = ox * a.stride - a.pad;
    const int n = n0 + r < a.N ? n0 + r : a.N - 1;
    const int8_t* brow = a.W + (size_t)n * a.ldw + q;
    const int ao = r * SP + q, bo = (BM + r) * SP + q;
    int ci = 0, kx = 0, ky = 0, kg = 0;  // the next slab's tap, channel offset and K offset
    v4i ra, rb;
    auto gload = [&]() {
        const int iy = iy0 + ky, ix = ix0 + kx;
        ra = v4i{0, 0, 0, 0};
        if (iy >= 0 && iy < a.H && ix >= 0 && ix < a.Wd)
            ra = *reinterpret_cast<const v4i*>(a.xq + ((size_t)iy * a.Wd + ix) * a.Cin + ci + q);
        rb = *reinterpret_cast<const v4i*>(brow + kg);
        kg += BK;
        ci += BK;
        if (ci == a.Cin) {
            ci = 0;
            if (++kx == a.k) {
                kx = 0;
                ++ky;
            }
        }
    };
    auto lstore = [&](int buf) {
        *reinterpret_cast<v4i*>(&sm[buf][ao]) = ra;
        *reinterpret_cast<v4i*>(&sm[buf][bo]) = rb;
    };
    v4i acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = v4i{0, 0, 0, 0};
    const int r16 = lane & 15, k16 = (lane >> 4) * 16;
    auto compute = [&](int buf) {
        const int8_t* sb = sm[buf];
        v4i af[2], bf[2];
#pragma unroll
        for (int i = 0; i < 2; i++) af[i] = *reinterpret_cast<const v4i*>(sb + (wm * 32 + i * 16 + r16) * SP + k16);
#pragma unroll
        for (int j = 0; j < 2; j++)
            bf[j] = *reinterpret_cast<const v4i*>(sb + (BM + wn * 32 + j * 16 + r16) * SP + k16);
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[j], af[i], acc[i][j], 0, 0, 0);
    };
    const int nk = a.K / BK;
    gload();
    lstore(0);
    if (nk > 1) gload();
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        compute(buf);
        if (kt + 1 < nk) {
            lstore(buf ^ 1);  // slab kt + 1, loaded during this compute
            if (kt + 2 < nk) gload();
        }
        __syncthreads();
    }
    // epilogue: fma((float)acc * ws[n], s, b[n]) per output (gemm_i8.cpp:278)
    const float s = *a.s;
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int mo = m0 + wm * 32 + i * 16 + r16;
        if (mo >= a.npix) continue;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int nb = n0 + wn * 32 + j * 16 + (lane >> 4) * 4;
            float v[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int nc = nb + c < a.N ? nb + c : a.N - 1;
                const float p = (float)acc[i][j][c] * a.wscale[nc];
                v[c] = fmaf(p, s, a.bias ? a.bias[nc] : 0.0f);
            }
            if (a.resid) {  // the block's residual add + ReLU
                const float* rr = a.resid + (size_t)mo * a.N + nb;
                if (nb + 4 <= a.N) {
                    const float4 r = *reinterpret_cast<const float4*>(rr);
                    v[0] = relu_gt(v[0] + r.x);
                    v[1] = relu_gt(v[1] + r.y);
                    v[2] = relu_gt(v[2] + r.z);
                    v[3] = relu_gt(v[3] + r.w);
                } else {
                    for (int c = 0; c < 4 && nb + c < a.N; c++) v[c] = relu_gt(v[c] + rr[c]);
                }
            } else if (a.act) {
#pragma unroll
                for (int c = 0; c < 4; c++) v[c] = act_relu(v[c]);
            }
#pragma unroll
            for (int c = 0; c < 4; c++)
                if (nb + c < a.N) mx = fmaxf(mx, fabsf(v[c]));
            float* o = a.out + (size_t)mo * a.N + nb;
            if (nb + 4 <= a.N) {
                *reinterpret_cast<float4*>(o) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
                for (int c = 0; c < 4 && nb + c < a.N; c++) o[c] = v[c];
            }
        }
    }
    if (a.omax) {  // one maximum per block
        __shared__ float red[4];
        mx = block_max(mx, red);
        if (tid == 0) a.omax[blockIdx.y * gridDim.x + blockIdx.x] = mx;
    }
}

// Inputs of at most 4 channels (the RGB stem): the input quantized once into
// one 32-bit word per pixel (its channels' bytes, the rest zero), and an
// implicit GEMM over K' = taps x 4 bytes. Zero bytes add nothing to the int32
// sums, so every sum - and, through the same epilogue, every output - equals
// the im2col path's. x [H * Wd, Cin] fp32 -> q [H * Wd] words; scale to *s_out.
// The same launch lays the weights out in K' order once: wc [N][KB / 4] words
// (tap t's word holds W[n][t * Cin + ci] in byte ci; zero past Cin and past
// the last tap).
__global__ __launch_bounds__(256) void conv_quant_c4_kernel(const float* __restrict__ x, int npx, int Cin,
                                                            uint32_t* __restrict__ q, const float* __restrict__ part,
                                                            int nparts, float clip, float* __restrict__ s_out,
                                                            const int8_t* __restrict__ W, int ldw, int kk, int N,
                                                            int KW, uint32_t* __restrict__ wc) {
    __shared__ float red[4];
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < N * KW; i += gridDim.x * blockDim.x) {
        const int n = i / KW, t = i - n * KW;
        uint32_t w = 0;
        if (t < kk)
            for (int c = 0; c < Cin; c++) w |= (uint32_t)(uint8_t)W[(size_t)n * ldw + t * Cin + c] << (8 * c);
        wc[i] = w;
    }
    const float s = fold_scale(part, nparts, clip, red);
    const float inv = 1.0f / s;
    if (blockIdx.x == 0 && threadIdx.x == 0) *s_out = s;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < npx; i += gridDim.x * blockDim.x) {
        const float* px = x + (size_t)i * Cin;
        uint32_t w = 0;
        for (int c = 0; c < Cin; c++) w |= (uint32_t)(q8(px[c], inv) & 0xff) << (8 * c);
        q[i] = w;
    }
}

struct C4Args {
    const uint32_t* xq;  // [H, Wd] words
    int H, Wd, Cin, k, stride, pad, Wout, npix;
    const int8_t* wc;    // [N][KS * 64] bytes in K' order (conv_quant_c4_kernel)
    const float* wscale;
    const float* bias;
    const float* s;
    float* out;          // [npix, N]
    int N, KS;           // KS: 64-byte K steps of K' = k * k * 4
    float* omax;         // or null: per block max(0, out) (the maxima after a ReLU)
};

// 64 pixels x 64 output channels per block, a wave per 16 pixels (4 MFMA
// fragments across the channels). The block first copies its channels'
// K'-ordered weights into LDS; each lane of a wave then gathers, per K step,
// the 4 words of its pixel's taps 16 s + 4 (l / 16) .. + 3 (zero outside the
// image) as its A fragment. The weight fragment goes first: lane l holds
// pixel l % 16 and the four consecutive channels 4 (l / 16) .. + 3, stored
// as one float4.
constexpr int kC4MaxKS = 4;  // K' <= 256 bytes: k <= 8
__global__ __launch_bounds__(256) void conv_i8_c4(C4Args a) {
    constexpr int SB = 64 * kC4MaxKS + 16;  // LDS row per channel, bytes
    __shared__ __attribute__((aligned(16))) int8_t wl[64 * SB];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * 64, kk = a.k * a.k, KB = a.KS * 64;
    for (int e = tid; e < 64 * a.KS * 4; e += 256) {  // 16-byte chunks: channel e / (4 KS), chunk e % (4 KS)
        const int c = e / (4 * a.KS), b = (e - c * 4 * a.KS) * 16;
        const int n = n0 + c < a.N ? n0 + c : a.N - 1;
        *reinterpret_cast<v4i*>(wl + c * SB + b) = *reinterpret_cast<const v4i*>(a.wc + (size_t)n * KB + b);
    }
    const int r16 = lane & 15, g = lane >> 4;
    const int m = blockIdx.y * 64 + wave * 16 + r16;
    const int mc = m < a.npix ? m : a.npix - 1;
    const int oy = mc / a.Wout, ox = mc - oy * a.Wout;
    const int iy0 = oy * a.stride - a.pad, ix0 = ox * a.stride - a.pad;
    v4i acc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) acc[j] = v4i{0, 0, 0, 0};
    __syncthreads();
    for (int st = 0; st < a.KS; st++) {
        int w4[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int t = st * 16 + g * 4 + u;
            const int ky = t / a.k, kx = t - ky * a.k;
            const int iy = iy0 + ky, ix = ix0 + kx;
            w4[u] = (t < kk && iy >= 0 && iy < a.H && ix >= 0 && ix < a.Wd) ? (int)a.xq[iy * a.Wd + ix] : 0;
        }
        const v4i af = v4i{w4[0], w4[1], w4[2], w4[3]};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const v4i bf = *reinterpret_cast<const v4i*>(wl + (j * 16 + r16) * SB + st * 64 + g * 16);
            acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf, af, acc[j], 0, 0, 0);
        }
    }
    // epilogue: fma((float)acc * ws[n], s, b[n]) per output (gemm_i8.cpp:278)
    const float s = *a.s;
    float mx = 0.0f;
    if (m < a.npix) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int nb = n0 + j * 16 + g * 4;
            if (nb >= a.N) break;
            float v[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int nc = nb + c < a.N ? nb + c : a.N - 1;
                const float p = (float)acc[j][c] * a.wscale[nc];
                v[c] = fmaf(p, s, a.bias ? a.bias[nc] : 0.0f);
            }
            float* o = a.out + (size_t)m * a.N + nb;
            if (nb + 4 <= a.N) {
                *reinterpret_cast<float4*>(o) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
                for (int c = 0; c < 4 && nb + c < a.N; c++) o[c] = v[c];
            }
#pragma unroll
            for (int c = 0; c < 4; c++)
                if (nb + c < a.N) mx = fmaxf(mx, v[c]);
        }
    }
    if (a.omax) {  // one maximum per block
        __shared__ float red[4];
        mx = block_max(mx, red);
        if (tid == 0) a.omax[blockIdx.y * gridDim.x + blockIdx.x] = mx;
    }
}

bool conv_implicit_on() {
    const char* e = std::getenv("VLA_HIP_CONV_IMPLICIT");
    return !(e && e[0] == '0' && e[1] == '\0');
}

// Convs over 64-channel multiples with more output pixels than the skinny
// GEMM's rows take the 32 x 64 LDS GEMM tile gathering A from the int8 map
// (VLA_HIP_CONV_LDS_IMPLICIT, read per call: 0 off, "all" at every pixel
// count)
int conv_lds_implicit_mode() {
    const char* e = std::getenv("VLA_HIP_CONV_LDS_IMPLICIT");
    if (e && e[0] == '0' && e[1] == '\0') return 0;
    if (e && std::strcmp(e, "all") == 0) return 2;
    return 1;
}

// The fewest 64 x 64 output tiles for which a k > 1 conv over 64-channel
// multiples that the LDS form does not take runs conv_i8_implicit
// (VLA_HIP_CONV_IMPLICIT_TILES, read per call; default 256, or never while
// the LDS form is on)
int64_t conv_implicit_tiles(int lds_mode) {
    const char* e = std::getenv("VLA_HIP_CONV_IMPLICIT_TILES");
    return e && *e ? std::atoll(e) : (lds_mode > 0 ? INT64_MAX : 256);
}

// The implicit forms' operands: 64-channel multiples, 16-byte rows.
bool implicit_operands(const ConvArgs& a) {
    return a.Cin % 64 == 0 && a.Cout % 4 == 0 && a.ldw % 16 == 0 && (reinterpret_cast<uintptr_t>(a.Wq) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.out) & 15) == 0 &&
           conv_implicit_on();
}

// Whether a takes a form that quantizes x once into the int8 map with
// npix row scales: the skinny kernel over the skinny GEMM's pixel counts
// (VLA_HIP_CONV_SKINNY_IMPLICIT=0: off), else the LDS tile (*skinny says
// which).
bool map_route(const ConvArgs& a, const ConvShape& c, bool* skinny) {
    const bool ok = implicit_operands(a);
    const int lds_mode = conv_lds_implicit_mode();
    const char* ske = std::getenv("VLA_HIP_CONV_SKINNY_IMPLICIT");
    const bool sk = ok && lds_mode == 1 && !(ske && ske[0] == '0' && ske[1] == '\0') &&
                    gemm_i8_conv_skinny_fits(c.npix, a.Cout);
    const bool lds = ok && !sk && lds_mode > 0 && (lds_mode == 2 || c.npix > 320);
    *skinny = sk;
    return sk || lds;
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
    // the A region holds the im2col rows, or the int8 input of the implicit
    // forms (one word per pixel up to 4 channels, then the K'-ordered weights)
    const size_t qin = Cin <= 4 ? ((size_t)H * Wd * 4 + 255) / 256 * 256 + (size_t)Cout * 256 : (size_t)H * Wd * Cin;
    const size_t arows = (size_t)c.npix * c.lda > qin ? (size_t)c.npix * c.lda : qin;
    c.work = (size_t)kAbsmaxBlocks * 4 + ((size_t)c.npix * 4 + 255) / 256 * 256 + (arows + 255) / 256 * 256 +
             c.split;
    return c;
}

int launch_conv2d_i8(const ConvArgs& a, hipStream_t st) {
    const ConvShape c = conv_shape(a.H, a.Wd, a.Cin, a.k, a.stride, a.pad, a.Cout);
    VLA_REQUIRE(a.x && a.out && a.Wq && a.wscale && a.work, "conv2d_i8: null buffer");
    VLA_REQUIRE(a.ldw >= kpad4(c.K) && a.ldw % 4 == 0, "conv2d_i8: bad weight rows");
    VLA_REQUIRE(a.work_bytes >= c.work, "conv2d_i8: workspace too small (vla_conv2d_i8_workspace_bytes)");
    VLA_REQUIRE((reinterpret_cast<uintptr_t>(a.work) & 255) == 0, "conv2d_i8: workspace must be 256-byte aligned");
    char* w = static_cast<char*>(a.work);
    if (a.xq_out) *a.xq_out = 0;
    // [block maxima: 512 floats][row scales: npix floats][im2col rows][split-K sums],
    // each 256-byte rounded
    float* part = reinterpret_cast<float*>(w);
    float* ascale = reinterpret_cast<float*>(w + (size_t)kAbsmaxBlocks * 4);
    int8_t* A = reinterpret_cast<int8_t*>(w + (size_t)kAbsmaxBlocks * 4 + ((size_t)c.npix * 4 + 255) / 256 * 256);

    int blocks;
    const float* maxima = part;
    if (a.in_part) {
        // the producer of x wrote its block maxima: no pass over x here
        VLA_REQUIRE(a.in_nparts > 0 && a.in_nparts <= kConvPartsFused, "conv2d_i8: 1..4096 producer block maxima");
        maxima = a.in_part;
        blocks = a.in_nparts;
    } else {
        const int64_t n = (int64_t)a.H * a.Wd * a.Cin;
        blocks = (int)((n + 4 * 256 * 4 - 1) / (4 * 256 * 4));
        blocks = blocks < 1 ? 1 : (blocks > kAbsmaxBlocks ? kAbsmaxBlocks : blocks);
        conv_absmax_kernel<<<blocks, 256, 0, st>>>(a.x, n, part);
        VLA_LAUNCH_CHECK();
    }

    const float clip = a.clip > 0.0f ? a.clip : clip_from_env();
    const int64_t tiles = (int64_t)((c.npix + 63) / 64) * ((a.Cout + 63) / 64);
    const bool impl_ok = implicit_operands(a);
    const int lds_mode = conv_lds_implicit_mode();
    bool skinny_take = false;
    const bool map_take = map_route(a, c, &skinny_take);
    const bool lds_take = map_take && !skinny_take;
    if (impl_ok && !map_take && (c.npix + 63) / 64 <= 65535 &&
        (a.k == 1 || tiles >= conv_implicit_tiles(lds_mode))) {
        const int64_t n4 = (int64_t)a.H * a.Wd * a.Cin / 4;
        const int qb = (int)((n4 + 255) / 256 < 2048 ? (n4 + 255) / 256 : 2048);
        conv_quant_kernel<<<qb, 256, 0, st>>>(reinterpret_cast<const float4*>(a.x), n4,
                                              reinterpret_cast<uint32_t*>(A), maxima, blocks, clip, ascale, 1);
        VLA_LAUNCH_CHECK();
        ImplicitArgs ia{A, a.H, a.Wd, a.Cin, a.k, a.stride, a.pad, c.Wout, c.npix, a.Wq, a.ldw, a.wscale,
                        a.bias, ascale, a.out, a.Cout, c.K};
        const dim3 grid((a.Cout + 63) / 64, (c.npix + 63) / 64);
        int parts = 0;
        if (a.out_part && !a.relu_maxima && (int64_t)grid.x * grid.y <= kConvPartsFused &&
            (!a.resid || (reinterpret_cast<uintptr_t>(a.resid) & 15) == 0)) {
            parts = (int)(grid.x * grid.y);
            ia.act = a.resid ? 0 : 1;
            ia.resid = a.resid;
            ia.omax = a.out_part;
        }
        conv_i8_implicit<<<grid, 256, 0, st>>>(ia);
        VLA_LAUNCH_CHECK();
        return parts;
    }

    if (a.Cin <= 4 && a.k * a.k * 4 <= 64 * kC4MaxKS && a.Cout % 4 == 0 &&
        (reinterpret_cast<uintptr_t>(a.out) & 15) == 0 && (c.npix + 63) / 64 <= 65535 && conv_implicit_on()) {
        const int npx = a.H * a.Wd, KS = (a.k * a.k * 4 + 63) / 64;
        const int qb = (npx + 255) / 256 < 2048 ? (npx + 255) / 256 : 2048;
        int8_t* wc = A + ((size_t)npx * 4 + 255) / 256 * 256;
        conv_quant_c4_kernel<<<qb, 256, 0, st>>>(a.x, npx, a.Cin, reinterpret_cast<uint32_t*>(A), maxima, blocks,
                                                 clip, ascale, a.Wq, a.ldw, a.k * a.k, a.Cout, KS * 16,
                                                 reinterpret_cast<uint32_t*>(wc));
        VLA_LAUNCH_CHECK();
        C4Args ca{reinterpret_cast<const uint32_t*>(A), a.H, a.Wd, a.Cin, a.k, a.stride, a.pad, c.Wout, c.npix,
                  wc, a.wscale, a.bias, ascale, a.out, a.Cout, KS, nullptr};
        const dim3 grid((a.Cout + 63) / 64, (c.npix + 63) / 64);
        int parts = 0;
        if (a.out_part && a.relu_maxima && !a.resid && (int64_t)grid.x * grid.y <= kConvPartsFused) {
            ca.omax = a.out_part;
            parts = (int)(grid.x * grid.y);
        }
        conv_i8_c4<<<grid, 256, 0, st>>>(ca);
        VLA_LAUNCH_CHECK();
        return parts;
    }

    if (lds_take || skinny_take) {
        if (!a.xq_in) {
            const int64_t n4 = (int64_t)a.H * a.Wd * a.Cin / 4;
            const int qb = (int)((n4 + 255) / 256 < 2048 ? (n4 + 255) / 256 : 2048);
            conv_quant_kernel<<<qb, 256, 0, st>>>(reinterpret_cast<const float4*>(a.x), n4,
                                                  reinterpret_cast<uint32_t*>(A), maxima, blocks, clip, ascale,
                                                  c.npix);
            VLA_LAUNCH_CHECK();
        }
        if (a.xq_out) *a.xq_out = 1;
        GemmArgs m{};
        m.A = A;
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
        m.cv_h = a.H;
        m.cv_w = a.Wd;
        m.cv_c = a.Cin;
        m.cv_k = a.k;
        m.cv_s = a.stride;
        m.cv_p = a.pad;
        m.cv_wo = c.Wout;
        const int64_t gblocks = (int64_t)((c.npix + 31) / 32) * ((a.Cout + 63) / 64);
        if (a.out_part && !a.relu_maxima && (skinny_take || gblocks <= kConvPartsFused) &&
            (!a.resid || (reinterpret_cast<uintptr_t>(a.resid) & 15) == 0)) {
            m.act = a.resid ? 0 : 1;
            m.resid = a.resid;
            m.omax = a.out_part;
        }
        return skinny_take ? launch_gemm_i8_conv_skinny_implicit(m, st) : launch_gemm_i8_conv_implicit(m, st);
    }

    Im2colArgs g{a.x, a.H, a.Wd, a.Cin, a.k, a.stride, a.pad, c.Wout, c.npix, c.K, c.lda, maxima, blocks,
                 clip, A, ascale};
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
    if (a.out_part && !a.relu_maxima) {
        m.act = a.resid ? 0 : 1;
        m.resid = a.resid;
        m.omax = a.out_part;
        const int parts = launch_gemm_i8_conv(m, st);
        if (parts > 0) return parts;
        m.act = 0;
        m.resid = nullptr;
        m.omax = nullptr;
    }
    launch_gemm_i8(m, st);
    return 0;
}

int launch_conv_pool_quant(const ConvArgs& a, const float* x, int H, int Wd, int k, int stride, int pad,
                           hipStream_t st) {
    if (!a.in_part || a.in_nparts <= 0 || a.in_nparts > kConvPartsFused || a.Cin % 4 != 0 || !a.x || !a.work ||
        (reinterpret_cast<uintptr_t>(x) & 15) != 0 || (reinterpret_cast<uintptr_t>(a.work) & 255) != 0)
        return 0;
    // every input pixel inside some window, so max(pooled) = max(0, max x)
    if (k < stride || pad < 0 || pad >= k || (int64_t)(a.H - 1) * stride - pad + k < H ||
        (int64_t)(a.Wd - 1) * stride - pad + k < Wd || (int64_t)(a.H - 1) * stride - pad >= H ||
        (int64_t)(a.Wd - 1) * stride - pad >= Wd)
        return 0;
    const ConvShape c = conv_shape(a.H, a.Wd, a.Cin, a.k, a.stride, a.pad, a.Cout);
    bool skinny = false;
    if (a.work_bytes < c.work || !map_route(a, c, &skinny)) return 0;
    const int64_t total4 = (int64_t)a.H * a.Wd * a.Cin / 4;
    if ((int64_t)H * Wd * a.Cin / 4 >= INT32_MAX || total4 >= INT32_MAX) return 0;
    char* w = static_cast<char*>(a.work);
    float* ascale = reinterpret_cast<float*>(w + (size_t)kAbsmaxBlocks * 4);
    uint32_t* A = reinterpret_cast<uint32_t*>(w + (size_t)kAbsmaxBlocks * 4 + ((size_t)c.npix * 4 + 255) / 256 * 256);
    const float clip = a.clip > 0.0f ? a.clip : clip_from_env();
    const int g = (int)((total4 + 255) / 256 < 2048 ? (total4 + 255) / 256 : 2048);
    conv_pool_quant4_kernel<<<g, 256, 0, st>>>(reinterpret_cast<float4*>(const_cast<float*>(a.x)),
                                               reinterpret_cast<const float4*>(x), H, Wd, a.Cin / 4, k, stride, pad,
                                               a.Wd, (int)total4, a.in_part, a.in_nparts, clip, A, ascale, c.npix);
    VLA_LAUNCH_CHECK();
    return 1;
}

}  // namespace hip
}  // namespace vla
