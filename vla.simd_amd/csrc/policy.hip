// policy.hip - the per-query glue of the model-level entry points around the
// transformers: camera preprocessing, token embedding lookup, state and action
// (un)normalization and the flow-matching update with real-time-chunking
// guidance. Each is a single pass over at most a few MB.
#include "common.h"

#include <algorithm>
#include <cmath>

#pragma clang fp contract(off)

namespace vla {
namespace hip {
namespace {

// src/preprocess/image.cpp:13-51: bilinear resize (half-pixel centres, edge
// clamp) into the bottom-right of an S x S canvas, padding -1, values
// v / 255 * 2 - 1, output CHW. One thread per output pixel of one view
// (blockIdx.y); the geometry comes from the host in the reference's double math.
__global__ __launch_bounds__(256) void resize_pad_kernel(float* __restrict__ dst, const uint8_t* __restrict__ src,
                                                         int h, int w, int S, int pad_h, int pad_w, double sy,
                                                         double sx) {
    const int64_t npx = (int64_t)S * S;
    const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= npx) return;
    const int view = blockIdx.y;
    const uint8_t* img = src + (int64_t)view * h * w * 3;
    float* out = dst + (int64_t)view * 3 * npx;
    const int y = (int)(p / S), x = (int)(p % S);
    const int oy = y - pad_h, ox = x - pad_w;
    if (oy < 0 || ox < 0) {
        out[p] = out[npx + p] = out[2 * npx + p] = -1.0f;
        return;
    }
    const double fy = (oy + 0.5) * sy - 0.5;
    int y0 = (int)floor(fy);
    const double dy = fy - y0;
    const int y1 = min(y0 + 1, h - 1);
    y0 = max(y0, 0);
    const double fx = (ox + 0.5) * sx - 0.5;
    int x0 = (int)floor(fx);
    const double dx = fx - x0;
    const int x1 = min(x0 + 1, w - 1);
    x0 = max(x0, 0);
    for (int c = 0; c < 3; c++) {
        const double p00 = img[((int64_t)y0 * w + x0) * 3 + c], p01 = img[((int64_t)y0 * w + x1) * 3 + c];
        const double p10 = img[((int64_t)y1 * w + x0) * 3 + c], p11 = img[((int64_t)y1 * w + x1) * 3 + c];
        const double v = (p00 * (1 - dx) + p01 * dx) * (1 - dy) + (p10 * (1 - dx) + p11 * dx) * dy;
        out[c * npx + p] = (float)(v / 255.0 * 2.0 - 1.0);
    }
}

// dst[t, :] = bf16(table[ids[t], :]) * scale (smolvla_model.cpp:232-238)
__global__ __launch_bounds__(256) void embed_bf16_kernel(float* __restrict__ dst, const uint16_t* __restrict__ table,
                                                         const int32_t* __restrict__ ids, int H, float scale) {
    const int t = blockIdx.y;
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= H) return;
    const uint16_t b = table[(int64_t)ids[t] * H + j];
    dst[(int64_t)t * H + j] = __uint_as_float((uint32_t)b << 16) * scale;
}

__global__ __launch_bounds__(256) void scale_kernel(float* __restrict__ x, int64_t n, float s) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        x[i] = x[i] * s;
}

// out [rows, ld] (columns >= cols untouched) from x [rows, cols]:
// (x - mean) / (std + eps) per column, rows >= n_real written as 0
__global__ __launch_bounds__(256) void normalize_pad_kernel(float* __restrict__ out, int ldo,
                                                            const float* __restrict__ x, int n_real, int rows,
                                                            int cols, const float* __restrict__ mean,
                                                            const float* __restrict__ stdv, float eps) {
    const int64_t n = (int64_t)rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int r = (int)(i / cols), c = (int)(i % cols);
        out[(int64_t)r * ldo + c] = r < n_real ? (x[i] - mean[c]) / (stdv[c] + eps) : 0.0f;
    }
}

// actions [rows, cols] = fma(a[r, c], std[c] + eps, mean[c]) from a [rows, lda]
// (smolvla_model.cpp:284-288 with the reference's contracted multiply-add)
__global__ __launch_bounds__(256) void unnormalize_kernel(float* __restrict__ out, const float* __restrict__ a,
                                                          int lda, int rows, int cols, const float* __restrict__ mean,
                                                          const float* __restrict__ stdv, float eps) {
    const int64_t n = (int64_t)rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int r = (int)(i / cols), c = (int)(i % cols);
        out[i] = fmaf(a[(int64_t)r * lda + c], stdv[c] + eps, mean[c]);
    }
}

// One Euler step with real-time-chunking guidance (action_expert.cpp:377-389):
// v -= gw * ((prev - (x - time * v)) * weights[r]); x += dt * v. gw is read
// from the device (one value per step) so a captured graph takes any
// max_guidance.
__global__ __launch_bounds__(256) void rtc_step_kernel(float* __restrict__ x, const float* __restrict__ v,
                                                       const float* __restrict__ prev,
                                                       const float* __restrict__ weights, const float* __restrict__ gw,
                                                       int step, int rows, int cols, float time, float dt) {
    const int64_t n = (int64_t)rows * cols;
    const float g = gw[step];
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int r = (int)(i / cols);
        float vt = v[i];
        const float xi = x[i];
        vt = fmaf(-g, (prev[i] - fmaf(-time, vt, xi)) * weights[r], vt);
        x[i] = fmaf(dt, vt, xi);
    }
}

int grid_for(int64_t n) {
    const int64_t b = (n + 255) / 256;
    return (int)(b < 4096 ? (b > 0 ? b : 1) : 4096);
}

}  // namespace

void resize_geometry(int h, int w, int S, int* pad_h, int* pad_w, double* sy, double* sx) {
    const double ratio = std::max((double)w / S, (double)h / S);
    int rw = (int)(w / ratio), rh = (int)(h / ratio);
    if (rw < 1) rw = 1;
    if (rh < 1) rh = 1;
    *pad_w = S - rw;
    *pad_h = S - rh;
    *sx = (double)w / rw;
    *sy = (double)h / rh;
}

void launch_resize_with_pad(float* dst, const uint8_t* src, int n_views, int h, int w, int S, hipStream_t st) {
    VLA_REQUIRE(dst && src && n_views > 0 && n_views < 65536 && h > 0 && w > 0 && S > 0,
                "resize_with_pad: bad arguments");
    int pad_h, pad_w;
    double sy, sx;
    resize_geometry(h, w, S, &pad_h, &pad_w, &sy, &sx);
    const int64_t npx = (int64_t)S * S;
    VLA_REQUIRE((npx + 255) / 256 < 2147483647LL, "resize_with_pad: canvas too large");
    resize_pad_kernel<<<dim3((unsigned)((npx + 255) / 256), n_views), 256, 0, st>>>(dst, src, h, w, S, pad_h, pad_w,
                                                                                   sy, sx);
    VLA_LAUNCH_CHECK();
}

void launch_embed_bf16(float* dst, const uint16_t* table, const int32_t* ids, int n, int H, float scale,
                       hipStream_t st) {
    VLA_REQUIRE(n >= 0 && n < 65536 && H > 0, "embed: bad arguments");
    if (n == 0) return;
    embed_bf16_kernel<<<dim3((H + 255) / 256, n), 256, 0, st>>>(dst, table, ids, H, scale);
    VLA_LAUNCH_CHECK();
}

void launch_scale(float* x, int64_t n, float s, hipStream_t st) {
    if (n <= 0) return;
    scale_kernel<<<grid_for(n), 256, 0, st>>>(x, n, s);
    VLA_LAUNCH_CHECK();
}

void launch_normalize_pad(float* out, int ldo, const float* x, int n_real, int rows, int cols, const float* mean,
                          const float* stdv, float eps, hipStream_t st) {
    VLA_REQUIRE(rows > 0 && cols > 0 && ldo >= cols && n_real >= 0, "normalize_pad: bad arguments");
    normalize_pad_kernel<<<grid_for((int64_t)rows * cols), 256, 0, st>>>(out, ldo, x, n_real, rows, cols, mean, stdv,
                                                                         eps);
    VLA_LAUNCH_CHECK();
}

void launch_unnormalize(float* out, const float* a, int lda, int rows, int cols, const float* mean,
                        const float* stdv, float eps, hipStream_t st) {
    VLA_REQUIRE(rows > 0 && cols > 0 && lda >= cols, "unnormalize: bad arguments");
    unnormalize_kernel<<<grid_for((int64_t)rows * cols), 256, 0, st>>>(out, a, lda, rows, cols, mean, stdv, eps);
    VLA_LAUNCH_CHECK();
}

void launch_rtc_step(float* x, const float* v, const float* prev, const float* weights, const float* gw, int step,
                     int rows, int cols, float time, float dt, hipStream_t st) {
    rtc_step_kernel<<<grid_for((int64_t)rows * cols), 256, 0, st>>>(x, v, prev, weights, gw, step, rows, cols, time,
                                                                    dt);
    VLA_LAUNCH_CHECK();
}

}  // namespace hip
}  // namespace vla
