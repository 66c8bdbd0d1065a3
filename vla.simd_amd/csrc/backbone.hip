// backbone.hip - the element-wise and gather kernels of ACT's ResNet-18 image
// backbone (src/models/act/resnet_backbone.cpp) and its camera/state
// processing (src/models/act/act_model.cpp). The convolutions themselves are
// GEMMs: fp32 ones as im2col + the fp32 matrix-core linear (linear_f32.hip),
// int8 ones (ACT_INT8 bit 32) as conv2d_i8 (conv.hip).
//
// Layouts are the reference's: images uint8 HWC, feature maps NHWC fp32
// [H, W, C], conv weights [Cout][k][k][Cin], so an im2col row is the taps
// [ky][kx][ci] of one output pixel (src/hal/common/conv.cpp:117-176).
#include "act.h"
#include "common.h"
#include "wave.h"

#include <cmath>

#pragma clang fp contract(off)

namespace vla {
namespace hip {
namespace {

// A producer's share of conv2d_i8's per-tensor scale: the block's max |v|
// over the values it wrote, stored at part[blockIdx.x] when part is given
// (uniform over the grid; every thread of the block reaches this point). The consuming conv2d_i8 folds these maxima
// instead of reading its input once more (max is order-free: the same scale).
__device__ __forceinline__ void store_block_absmax(float m, float* __restrict__ part) {
    if (!part) return;
    __shared__ float red[4];
    m = wave_max_f32(m);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        float v = 0.0f;
        for (int w = 0; w < (int)(blockDim.x >> 6); w++) v = fmaxf(v, red[w]);
        part[blockIdx.x] = v;
    }
}

// act_model.cpp:109-123: (pixel / 255 - mean[c]) / (std[c] + eps), the
// lerobot NormalizerProcessorStep order, one camera's [npx, 3] block per
// blockIdx.y (stats [n_cams][3]).
__global__ __launch_bounds__(256) void normalize_u8_kernel(float* __restrict__ out, const uint8_t* __restrict__ img,
                                                           int64_t npx3, const float* __restrict__ mean,
                                                           const float* __restrict__ stdv, float eps,
                                                           float* __restrict__ part) {
    const int cam = blockIdx.y;
    const uint8_t* src = img + (int64_t)cam * npx3;
    float* dst = out + (int64_t)cam * npx3;
    const float* m = mean + cam * 3;
    const float* s = stdv + cam * 3;
    float mx = 0.0f;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < npx3; i += (int64_t)gridDim.x * blockDim.x) {
        const int c = (int)(i % 3);
        const float v = ((float)src[i] / 255.0f - m[c]) / (s[c] + eps);
        dst[i] = v;
        mx = fmaxf(mx, fabsf(v));
    }
    // camera c's maxima at part[c * kConvPartMax ...]
    store_block_absmax(mx, part ? part + (size_t)cam * kConvPartMax : nullptr);
}

// im2col of an NHWC map for a k x k conv: row p = output pixel (oy, ox),
// column (ky * k + kx) * Cin + ci = x[oy*stride - pad + ky][ox*stride - pad + kx][ci],
// zero outside the image; columns [K, ldc) are left alone (never read).
__global__ __launch_bounds__(256) void im2col_f32_kernel(float* __restrict__ col, int ldc, const float* __restrict__ x,
                                                         int H, int Wd, int Cin, int k, int stride, int pad, int Wout,
                                                         int64_t total) {
    const int K = k * k * Cin;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t p = e / K;
        const int r = (int)(e - p * K);
        const int ci = r % Cin, t = r / Cin, kx = t % k, ky = t / k;
        const int oy = (int)(p / Wout), ox = (int)(p % Wout);
        const int iy = oy * stride - pad + ky, ix = ox * stride - pad + kx;
        const bool in = iy >= 0 && iy < H && ix >= 0 && ix < Wd;
        col[p * ldc + r] = in ? x[((int64_t)iy * Wd + ix) * Cin + ci] : 0.0f;
    }
}

// The same columns when Cin % 4 == 0 (every layer after a stem): one thread
// copies 4 channels of one tap as a float4 (they never straddle two taps),
// with 32-bit index math; values identical to im2col_f32_kernel's.
__global__ __launch_bounds__(256) void im2col_f32x4_kernel(float* __restrict__ col, int ldc,
                                                           const float* __restrict__ x, int H, int Wd, int Cin, int k,
                                                           int stride, int pad, int Wout, int K4, int total) {
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
        const int p = e / K4, r = 4 * (e - p * K4);
        const int t = r / Cin, ci = r - t * Cin;
        const int ky = t / k, kx = t - ky * k;
        const int oy = p / Wout, ox = p - oy * Wout;
        const int iy = oy * stride - pad + ky, ix = ox * stride - pad + kx;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (iy >= 0 && iy < H && ix >= 0 && ix < Wd)
            v = *reinterpret_cast<const float4*>(x + ((size_t)iy * Wd + ix) * Cin + ci);
        *reinterpret_cast<float4*>(col + (size_t)p * ldc + r) = v;
    }
}

// The same columns for any Cin (the 3-channel stem) with K <= 256 and 32-bit
// sizes: a wave per output pixel, its lanes walking the row (coalesced
// stores), each lane's taps (ky, kx, ci) decomposed once; values identical
// to im2col_f32_kernel's.
__global__ __launch_bounds__(256) void im2col_f32_rows_kernel(float* __restrict__ col, int ldc,
                                                              const float* __restrict__ x, int H, int Wd, int Cin,
                                                              int k, int stride, int pad, int Wout, int npix) {
    const int lane = threadIdx.x & 63;
    const int K = k * k * Cin;
    int dy[4], dx[4], ci[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int r = lane + 64 * j, t = r / Cin;
        ci[j] = r - t * Cin;
        dy[j] = t / k;
        dx[j] = t - dy[j] * k;
    }
    for (int p = blockIdx.x * 4 + (threadIdx.x >> 6); p < npix; p += gridDim.x * 4) {
        const int oy = p / Wout, ox = p - oy * Wout;
        const int y0 = oy * stride - pad, x0 = ox * stride - pad;
        float* crow = col + (size_t)p * ldc;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = lane + 64 * j;
            if (r >= K) break;
            const int iy = y0 + dy[j], ix = x0 + dx[j];
            const bool in = iy >= 0 && iy < H && ix >= 0 && ix < Wd;
            crow[r] = in ? x[(iy * Wd + ix) * Cin + ci[j]] : 0.0f;
        }
    }
}

// maxpool2d_relu (src/hal/common/conv.cpp:192-224): padded taps count as -inf,
// then the folded ReLU (!(v > 0) -> 0).
__global__ __launch_bounds__(256) void maxpool_relu_kernel(float* __restrict__ out, const float* __restrict__ x, int H,
                                                           int Wd, int C, int k, int stride, int pad, int Hout,
                                                           int Wout, float* __restrict__ part) {
    const int64_t total = (int64_t)Hout * Wout * C;
    float mx = 0.0f;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        const int c = (int)(e % C);
        const int64_t p = e / C;
        const int oy = (int)(p / Wout), ox = (int)(p % Wout);
        float o = -INFINITY;
        for (int ky = 0; ky < k; ky++) {
            const int iy = oy * stride - pad + ky;
            if (iy < 0 || iy >= H) continue;
            for (int kx = 0; kx < k; kx++) {
                const int ix = ox * stride - pad + kx;
                if (ix < 0 || ix >= Wd) continue;
                const float v = x[((int64_t)iy * Wd + ix) * C + c];
                o = v > o ? v : o;
            }
        }
        const float r = o > 0.0f ? o : 0.0f;
        out[e] = r;
        mx = fmaxf(mx, r);
    }
    store_block_absmax(mx, part);
}

// the basic block's tail (resnet_backbone.cpp:296-303): o = max(o + identity, 0)
// as v > 0 ? v : 0
__global__ __launch_bounds__(256) void add_relu_kernel(float* __restrict__ o, const float* __restrict__ idn, int64_t n,
                                                      float* __restrict__ part) {
    float mx = 0.0f;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float v = o[i] + idn[i];
        const float r = v > 0.0f ? v : 0.0f;
        o[i] = r;
        mx = fmaxf(mx, r);
    }
    store_block_absmax(mx, part);
}

// IMPACT's FiLM point after a basic block (resnet_backbone.cpp:276-290):
// v = o + idn, o = (1 + gamma[c]) * relu(v) + beta[c] over NHWC maps of C
// channels; the multiply-add is one fused operation, as the reference's
// -ffp-contract=fast build emits it. The block maxima are of |o| (the
// modulated map can go negative).
__global__ __launch_bounds__(256) void add_relu_film_kernel(float* __restrict__ o, const float* __restrict__ idn,
                                                           int64_t n, int C, const float* __restrict__ gamma,
                                                           const float* __restrict__ beta, float* __restrict__ part) {
    float mx = 0.0f;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int c = (int)(i % C);
        const float v = o[i] + idn[i];
        const float r = v > 0.0f ? v : 0.0f;
        const float y = fmaf(1.0f + gamma[c], r, beta[c]);
        o[i] = y;
        mx = fmaxf(mx, fabsf(y));
    }
    store_block_absmax(mx, part);
}

// The same four ops over float4 groups (C % 4 == 0, 16-byte aligned maps, a
// thread per output pixel and 4 channels, 32-bit indices): the per-element
// expressions above, so every stored float and block maximum's max is the
// same; the scalar forms loop over 64-bit element indices and stay for the
// shapes these do not take.
__device__ __forceinline__ float pool_max(float v, float o) { return v > o ? v : o; }

__global__ __launch_bounds__(256) void maxpool_relu4_kernel(float4* __restrict__ out, const float4* __restrict__ x, int H,
                                                            int Wd, int C4, int k, int stride, int pad, int Wout,
                                                            int total4, float* __restrict__ part) {
    float mx = 0.0f;
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
                o.x = pool_max(v.x, o.x);
                o.y = pool_max(v.y, o.y);
                o.z = pool_max(v.z, o.z);
                o.w = pool_max(v.w, o.w);
            }
        }
        const float4 r = make_float4(relu_gt(o.x), relu_gt(o.y), relu_gt(o.z), relu_gt(o.w));
        out[e] = r;
        mx = fmaxf(fmaxf(mx, fmaxf(r.x, r.y)), fmaxf(r.z, r.w));
    }
    store_block_absmax(mx, part);
}

__global__ __launch_bounds__(256) void add_relu4_kernel(float4* __restrict__ o, const float4* __restrict__ idn, int n4,
                                                        float* __restrict__ part) {
    float mx = 0.0f;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += gridDim.x * blockDim.x) {
        const float4 a = o[i], b = idn[i];
        const float4 r = make_float4(relu_gt(a.x + b.x), relu_gt(a.y + b.y), relu_gt(a.z + b.z), relu_gt(a.w + b.w));
        o[i] = r;
        mx = fmaxf(fmaxf(mx, fmaxf(r.x, r.y)), fmaxf(r.z, r.w));
    }
    store_block_absmax(mx, part);
}

__global__ __launch_bounds__(256) void relu4_kernel(float4* __restrict__ x, int n4, float* __restrict__ part) {
    float mx = 0.0f;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += gridDim.x * blockDim.x) {
        float4 v = x[i];
        if (v.x < 0.0f || v.y < 0.0f || v.z < 0.0f || v.w < 0.0f) {
            if (v.x < 0.0f) v.x = 0.0f;
            if (v.y < 0.0f) v.y = 0.0f;
            if (v.z < 0.0f) v.z = 0.0f;
            if (v.w < 0.0f) v.w = 0.0f;
            x[i] = v;
        }
        mx = fmaxf(fmaxf(mx, fmaxf(fabsf(v.x), fabsf(v.y))), fmaxf(fabsf(v.z), fabsf(v.w)));
    }
    store_block_absmax(mx, part);
}

__global__ __launch_bounds__(256) void add_relu_film4_kernel(float4* __restrict__ o, const float4* __restrict__ idn,
                                                             int n4, int C4, const float4* __restrict__ gamma,
                                                             const float4* __restrict__ beta, float* __restrict__ part) {
    float mx = 0.0f;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += gridDim.x * blockDim.x) {
        const int c4 = i % C4;
        const float4 a = o[i], b = idn[i], g = gamma[c4], be = beta[c4];
        float4 y;
        y.x = fmaf(1.0f + g.x, relu_gt(a.x + b.x), be.x);
        y.y = fmaf(1.0f + g.y, relu_gt(a.y + b.y), be.y);
        y.z = fmaf(1.0f + g.z, relu_gt(a.z + b.z), be.z);
        y.w = fmaf(1.0f + g.w, relu_gt(a.w + b.w), be.w);
        o[i] = y;
        mx = fmaxf(fmaxf(mx, fmaxf(fabsf(y.x), fabsf(y.y))), fmaxf(fabsf(y.z), fabsf(y.w)));
    }
    store_block_absmax(mx, part);
}

// relu in place as the reference's relu (eltwise.cpp:209-215): x < 0 -> 0
__global__ __launch_bounds__(256) void relu_kernel(float* __restrict__ x, int64_t n, float* __restrict__ part) {
    float mx = 0.0f;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        float v = x[i];
        if (v < 0.0f) x[i] = v = 0.0f;
        mx = fmaxf(mx, fabsf(v));
    }
    store_block_absmax(mx, part);
}

// per-column affine of [rows, cols]: mode 0 (x - a[c]) / (b[c] + eps) (the
// state normalization, act_model.cpp:145-147), mode 1 fma(x, b[c], a[c]) (the
// action un-normalization v * std + mean, :152-157, which the reference's
// -ffp-contract=fast build emits as one fma)
__global__ __launch_bounds__(256) void col_affine_kernel(float* __restrict__ out, const float* __restrict__ x, int rows,
                                                         int cols, const float* __restrict__ a,
                                                         const float* __restrict__ b, float eps, int mode) {
    const int64_t n = (int64_t)rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int c = (int)(i % cols);
        out[i] = mode == 0 ? (x[i] - a[c]) / (b[c] + eps) : fmaf(x[i], b[c], a[c]);
    }
}

int grid_for(int64_t n) {
    const int64_t b = (n + 255) / 256;
    return (int)(b < 8192 ? (b > 0 ? b : 1) : 8192);
}

}  // namespace

// grid of a producer that writes block maxima: at most kConvPartMax blocks
static int part_grid(int64_t n, const float* part, int max_parts = kConvPartMax) {
    const int g = grid_for(n);
    return part && g > max_parts ? max_parts : g;
}

int launch_normalize_u8(float* out, const uint8_t* img, int n_cams, int64_t npx, const float* mean,
                        const float* stdv, float eps, hipStream_t st, float* part) {
    VLA_REQUIRE(n_cams > 0 && npx > 0 && out && img && mean && stdv, "normalize: bad arguments");
    const int gx = grid_for(npx * 3) < (part ? kConvPartMax : 1024) ? grid_for(npx * 3) : (part ? kConvPartMax : 1024);
    normalize_u8_kernel<<<dim3(gx, n_cams), 256, 0, st>>>(out, img, npx * 3, mean, stdv, eps, part);
    VLA_LAUNCH_CHECK();
    return gx;
}

void launch_im2col_f32(float* col, int ldc, const float* x, int H, int Wd, int Cin, int k, int stride, int pad,
                       int Hout, int Wout, hipStream_t st) {
    const int64_t K = (int64_t)k * k * Cin;
    VLA_REQUIRE(ldc >= K && col && x, "im2col: bad arguments");
    const int64_t total = (int64_t)Hout * Wout * K;
    if (Cin % 4 == 0 && ldc % 4 == 0 && total / 4 < INT32_MAX && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
        (reinterpret_cast<uintptr_t>(col) & 15) == 0) {
        const int64_t t4 = total / 4;
        im2col_f32x4_kernel<<<grid_for(t4), 256, 0, st>>>(col, ldc, x, H, Wd, Cin, k, stride, pad, Wout, (int)(K / 4),
                                                          (int)t4);
    } else if (K <= 256 && (int64_t)H * Wd * Cin < INT32_MAX && (int64_t)Hout * Wout < INT32_MAX) {
        const int npix = Hout * Wout;
        const int blocks = (npix + 3) / 4 < 16384 ? (npix + 3) / 4 : 16384;
        im2col_f32_rows_kernel<<<blocks, 256, 0, st>>>(col, ldc, x, H, Wd, Cin, k, stride, pad, Wout, npix);
    } else {
        im2col_f32_kernel<<<grid_for(total), 256, 0, st>>>(col, ldc, x, H, Wd, Cin, k, stride, pad, Wout, total);
    }
    VLA_LAUNCH_CHECK();
}

int launch_maxpool_relu(float* out, const float* x, int H, int Wd, int C, int k, int stride, int pad, int Hout,
                        int Wout, hipStream_t st, float* part, int max_parts) {
    VLA_REQUIRE(out && x && Hout > 0 && Wout > 0 && C > 0, "maxpool: bad arguments");
    const int64_t total = (int64_t)Hout * Wout * C;
    if (C % 4 == 0 && aligned(out, 16) && aligned(x, 16) && (int64_t)H * Wd * C / 4 < INT32_MAX &&
        total / 4 < INT32_MAX) {
        const int g = part_grid(total / 4, part, max_parts);
        maxpool_relu4_kernel<<<g, 256, 0, st>>>(reinterpret_cast<float4*>(out), reinterpret_cast<const float4*>(x), H,
                                                 Wd, C / 4, k, stride, pad, Wout, (int)(total / 4), part);
        VLA_LAUNCH_CHECK();
        return g;
    }
    const int g = part_grid(total, part, max_parts);
    maxpool_relu_kernel<<<g, 256, 0, st>>>(out, x, H, Wd, C, k, stride, pad, Hout, Wout, part);
    VLA_LAUNCH_CHECK();
    return g;
}

int launch_add_relu(float* o, const float* idn, int64_t n, hipStream_t st, float* part) {
    if (n % 4 == 0 && n / 4 < INT32_MAX && aligned(o, 16) && aligned(idn, 16)) {
        const int g = part_grid(n / 4, part);
        add_relu4_kernel<<<g, 256, 0, st>>>(reinterpret_cast<float4*>(o), reinterpret_cast<const float4*>(idn),
                                            (int)(n / 4), part);
        VLA_LAUNCH_CHECK();
        return g;
    }
    const int g = part_grid(n, part);
    add_relu_kernel<<<g, 256, 0, st>>>(o, idn, n, part);
    VLA_LAUNCH_CHECK();
    return g;
}

int launch_add_relu_film(float* o, const float* idn, int64_t n, int C, const float* gamma, const float* beta,
                         hipStream_t st, float* part) {
    VLA_REQUIRE(n > 0 && C > 0 && n % C == 0 && o && idn && gamma && beta, "add_relu_film: bad arguments");
    if (C % 4 == 0 && n / 4 < INT32_MAX && aligned(o, 16) && aligned(idn, 16) && aligned(gamma, 16) &&
        aligned(beta, 16)) {
        const int g = part_grid(n / 4, part);
        add_relu_film4_kernel<<<g, 256, 0, st>>>(reinterpret_cast<float4*>(o), reinterpret_cast<const float4*>(idn),
                                                 (int)(n / 4), C / 4, reinterpret_cast<const float4*>(gamma),
                                                 reinterpret_cast<const float4*>(beta), part);
        VLA_LAUNCH_CHECK();
        return g;
    }
    const int g = part_grid(n, part);
    add_relu_film_kernel<<<g, 256, 0, st>>>(o, idn, n, C, gamma, beta, part);
    VLA_LAUNCH_CHECK();
    return g;
}

int launch_relu_inplace(float* x, int64_t n, hipStream_t st, float* part) {
    if (n % 4 == 0 && n / 4 < INT32_MAX && aligned(x, 16)) {
        const int g = part_grid(n / 4, part);
        relu4_kernel<<<g, 256, 0, st>>>(reinterpret_cast<float4*>(x), (int)(n / 4), part);
        VLA_LAUNCH_CHECK();
        return g;
    }
    const int g = part_grid(n, part);
    relu_kernel<<<g, 256, 0, st>>>(x, n, part);
    VLA_LAUNCH_CHECK();
    return g;
}

void launch_col_affine(float* out, const float* x, int rows, int cols, const float* a, const float* b, float eps,
                       int mode, hipStream_t st) {
    VLA_REQUIRE(rows > 0 && cols > 0 && out && x && a && b, "col_affine: bad arguments");
    col_affine_kernel<<<grid_for((int64_t)rows * cols), 256, 0, st>>>(out, x, rows, cols, a, b, eps, mode);
    VLA_LAUNCH_CHECK();
}

}  // namespace hip
}  // namespace vla
