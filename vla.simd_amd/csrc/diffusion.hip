// diffusion.hip - Diffusion Policy's per-step and per-query kernels around its
// GEMMs: the UNet's GroupNorm + Mish with the FiLM or the residual folded in,
// the rgb encoders' spatial soft-argmax, the camera crop + normalization, the
// MIN_MAX state and action maps, the conditioning rows and the DDPM / DDIM
// update. The UNet works on [T, C] channel-last rows (T <= the horizon), so
// each of these is a few microseconds of latency, not bandwidth.
#include "common.h"
#include "wave.h"

#include <cmath>

#pragma clang fp contract(off)

namespace vla {
namespace hip {
namespace {

// mish with the reference's default (SIMD) form (eltwise.cpp:217-236):
// e = exp(min(v, 20)), v * (e (e + 2)) / (e (e + 2) + 2) = v tanh(softplus(v))
__device__ __forceinline__ float mish_f(float v) {
    const float e = expf(fminf(v, 20.0f));
    const float m = e * (e + 2.0f);
    return v * (m / (m + 2.0f));
}

constexpr int kGnThreads = 256;
constexpr int kGnRegs = 16;  // elements per thread held in registers (groups of <= 4096 values)

// groupnorm (conv.cpp:227-318) over the T rows of one group's gc channels,
// then mish, then at most one of: the FiLM y = fmaf(sc[c], y, bi[c])
// (scale) or y + bi[c] (bias only) of DPResBlock::forward
// (unet1d.cpp:186-199), or the residual y + res[t, c] (:203-211); stored to
// out and, when out2 is set, to out2 as well (the UNet's skip and
// concatenation copies). One block per group: each thread sums its
// elements' shifted values (shift: the group's first value) in double, the
// waves reduce through DPP, the four wave sums go through LDS in a fixed
// order; mean and variance are double, as the reference's. out may be x.
template <bool REG>
__global__ __launch_bounds__(kGnThreads) void gn_mish_kernel(float* out, int ldo, float* out2, int ldo2,
                                                             const float* x, int ldx, int T, int gc,
                                                             const float* __restrict__ scale,
                                                             const float* __restrict__ bias, float eps,
                                                             const float* __restrict__ sc,
                                                             const float* __restrict__ bi,
                                                             const float* __restrict__ res, int ldr) {
    __shared__ double red[2][kGnThreads / 64];
    const int tid = threadIdx.x, c0 = blockIdx.x * gc, n = T * gc;
    const double K = (double)x[c0];
    double s1 = 0.0, s2 = 0.0;
    // REG: the elements and everything their outputs read besides the
    // statistics (norm scale / bias, FiLM, residual), loaded up front so
    // those loads overlap the reduction
    float v[REG ? kGnRegs : 1], ps[REG ? kGnRegs : 1], pb[REG ? kGnRegs : 1], pf[REG ? kGnRegs : 1],
        pr[REG ? kGnRegs : 1];
    if (REG) {
#pragma unroll
        for (int i = 0; i < kGnRegs; i++) {
            const int e = tid + i * kGnThreads;
            v[i] = ps[i] = pb[i] = pf[i] = pr[i] = 0.0f;
            if (e < n) {
                const int t = e / gc, c = c0 + (e - t * gc);
                v[i] = x[(size_t)t * ldx + c];
                ps[i] = scale[c];
                pb[i] = bias[c];
                if (sc) pf[i] = sc[c];
                if (bi) pr[i] = bi[c];
                if (res) pr[i] = res[(size_t)t * ldr + c];
            }
        }
#pragma unroll
        for (int i = 0; i < kGnRegs; i++)
            if (tid + i * kGnThreads < n) {
                const double d = (double)v[i] - K;
                s1 += d;
                s2 += d * d;
            }
    } else {
        for (int e = tid; e < n; e += kGnThreads) {
            const int t = e / gc;
            const double d = (double)x[(size_t)t * ldx + c0 + (e - t * gc)] - K;
            s1 += d;
            s2 += d * d;
        }
    }
    s1 = wave_sum_f64(s1);
    s2 = wave_sum_f64(s2);
    if ((tid & 63) == 0) {
        red[0][tid >> 6] = s1;
        red[1][tid >> 6] = s2;
    }
    __syncthreads();
    double S1 = 0.0, S2 = 0.0;
#pragma unroll
    for (int w = 0; w < kGnThreads / 64; w++) {
        S1 += red[0][w];
        S2 += red[1][w];
    }
    // sum (x - mean)^2 = sum (x - K)^2 - n (mean - K)^2
    const double md = S1 / n, mean = K + md;
    const double inv = 1.0 / sqrt(fmax(S2 / n - md * md, 0.0) + (double)eps);
    // y = mish(x A + B), A = inv scale, B = bias - mean inv scale (double,
    // then float, as the reference's), then the FiLM / residual term
    auto apply = [&](int e, float xv, float gs, float gb, float fs, float fb) {
        const int t = e / gc, c = c0 + (e - t * gc);
        const float A = (float)(inv * (double)gs);
        const float B = (float)((double)gb - mean * inv * (double)gs);
        float y = mish_f(fmaf(xv, A, B));
        if (sc) y = fmaf(fs, y, fb);
        else if (bi || res) y = y + fb;
        out[(size_t)t * ldo + c] = y;
        if (out2) out2[(size_t)t * ldo2 + c] = y;
    };
    if (REG) {
#pragma unroll
        for (int i = 0; i < kGnRegs; i++)
            if (tid + i * kGnThreads < n) apply(tid + i * kGnThreads, v[i], ps[i], pb[i], pf[i], pr[i]);
    } else {
        for (int e = tid; e < n; e += kGnThreads) {
            const int t = e / gc, c = c0 + (e - t * gc);
            apply(e, x[(size_t)t * ldx + c], scale[c], bias[c], sc ? sc[c] : 0.0f,
                  res ? res[(size_t)t * ldr + c] : bi ? bi[c] : 0.0f);
        }
    }
}

// spatial_softmax (conv.cpp:398-420): per keypoint channel c of x [npx, C],
// the softmax over the pixels with the max shift, then the expected grid
// coordinate; one thread per channel walks the pixels in order, as the
// reference's loop does. out [C, 2].
__global__ __launch_bounds__(64) void spatial_softmax_kernel(float* __restrict__ out, const float* __restrict__ x,
                                                             const float* __restrict__ grid, int npx, int C) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C) return;
    float m = -INFINITY;
    for (int p = 0; p < npx; p++) m = fmaxf(m, x[(size_t)p * C + c]);
    float sum = 0.0f, ex = 0.0f, ey = 0.0f;
    for (int p = 0; p < npx; p++) {
        const float e = expf(x[(size_t)p * C + c] - m);
        sum += e;
        ex = fmaf(e, grid[2 * p], ex);
        ey = fmaf(e, grid[2 * p + 1], ey);
    }
    const float inv = 1.0f / sum;
    out[2 * c] = ex * inv;
    out[2 * c + 1] = ey * inv;
}

// DiffusionModel::preprocess (diffusion_model.cpp:178-201): the centre crop of
// an [H, W, 3] uint8 frame at (top, left), (v / 255 - mean) / (std + eps)
__global__ __launch_bounds__(256) void crop_normalize_kernel(float* __restrict__ out,
                                                             const uint8_t* __restrict__ img, int W, int top,
                                                             int left, int oh, int ow,
                                                             const float* __restrict__ mean,
                                                             const float* __restrict__ stdv, float eps) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t n = (int64_t)oh * ow * 3;
    if (i >= n) return;
    const int c = (int)(i % 3);
    const int64_t p = i / 3;
    const int y = (int)(p / ow), xx = (int)(p % ow);
    const float v = (float)img[((int64_t)(y + top) * W + left + xx) * 3 + c];
    out[i] = (v / 255.0f - mean[c]) / (stdv[c] + eps);
}

// the global conditioning of DiffusionModel::predict (:209-262): per
// observation step s, [state normalized to [-1, 1] (MIN_MAX) | the cameras'
// features], feats [steps * n_cams, F] in (step, camera) order
__global__ __launch_bounds__(256) void gcond_kernel(float* __restrict__ g, const float* __restrict__ state,
                                                    const float* __restrict__ smin, const float* __restrict__ smax,
                                                    const float* __restrict__ feats, int steps, int sd, int n_cams,
                                                    int F, float eps) {
    const int per = sd + n_cams * F;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= steps * per) return;
    const int s = i / per, k = i - s * per;
    if (k < sd) {
        const float den = smax[k] - smin[k];
        const float d = den == 0.0f ? eps : den;
        g[i] = 2.0f * (state[(size_t)s * sd + k] - smin[k]) / d - 1.0f;
    } else {
        g[i] = feats[(size_t)s * n_cams * F + (k - sd)];
    }
}

// the Mish of every block's cond encoder, per denoising step i:
// gm [steps, D + G] = [mish'd time embedding of step i (temb [steps, D]) | mish(gcond [G])]
__global__ __launch_bounds__(256) void cond_rows_kernel(float* __restrict__ gm, const float* __restrict__ temb,
                                                        const float* __restrict__ gcond, int steps, int D, int G) {
    const int CD = D + G;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)steps * CD) return;
    const int s = (int)(i / CD), k = (int)(i - (int64_t)s * CD);
    gm[i] = k < D ? temb[(size_t)s * D + k] : mish_f(gcond[k - D]);
}

__global__ __launch_bounds__(256) void mish_kernel(float* __restrict__ x, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = mish_f(x[i]);
}

// DPNoiseScheduler::step (scheduler.cpp:77-121) in double, coefficients from
// the host: x0 = clip((x - sqrt_bp e) / sqrt_ap); DDPM x = c0 x0 + c1 x
// (+ var z); DDIM x = sqrt_app x0 + dir e
struct SchedStep {
    double sqrt_ap, sqrt_bp, c0, c1, var, lo, hi;
    int ddim, clip, noise;
};
__global__ __launch_bounds__(256) void sched_step_kernel(float* __restrict__ x, const float* __restrict__ e,
                                                         const float* __restrict__ z, int n, SchedStep p) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const double xs = (double)x[i], ev = (double)e[i];
    double x0 = (xs - p.sqrt_bp * ev) / p.sqrt_ap;
    if (p.clip) x0 = fmin(p.hi, fmax(p.lo, x0));
    double v;
    if (p.ddim) {
        v = p.c0 * x0 + p.c1 * ev;
    } else {
        v = p.c0 * x0 + p.c1 * xs;
        if (p.noise) v += p.var * (double)z[i];
    }
    x[i] = (float)v;
}

// the executed slice of the horizon (rows start.. of x [horizon, A]) and the
// MIN_MAX un-normalization (s + 1) / 2 * d + min (diffusion_model.cpp:264-281)
__global__ __launch_bounds__(256) void dp_actions_kernel(float* __restrict__ out, const float* __restrict__ x,
                                                         int start, int chunk, int A,
                                                         const float* __restrict__ amin,
                                                         const float* __restrict__ amax, float eps, int unnorm) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= chunk * A) return;
    const int t = i / A, k = i - t * A;
    const float v = x[(size_t)(start + t) * A + k];
    if (unnorm) {
        const float den = amax[k] - amin[k];
        const float d = den == 0.0f ? eps : den;
        out[i] = fmaf((v + 1.0f) / 2.0f, d, amin[k]);
    } else {
        out[i] = v;
    }
}

int blocks_for(int64_t n) { return (int)((n + 255) / 256); }

}  // namespace

void launch_dp_gn_mish(float* out, int ldo, const float* x, int ldx, int T, int C, int groups, const float* scale,
                       const float* bias, float eps, const float* film_scale, const float* film_bias,
                       const float* res, int ldr, hipStream_t st, float* out2, int ldo2) {
    VLA_REQUIRE(out && x && scale && bias && T > 0 && C > 0 && groups > 0 && C % groups == 0,
                "dp_gn_mish: bad shape");
    const int gc = C / groups;
    VLA_REQUIRE(gc <= kDpGnMaxGroup && (int64_t)T * gc < INT32_MAX && ldx >= C && ldo >= C &&
                    (!res || ldr >= C) && (!out2 || ldo2 >= C),
                "dp_gn_mish: bad strides");
    VLA_REQUIRE(!film_scale || film_bias, "dp_gn_mish: FiLM scale without bias");
    VLA_REQUIRE(!(film_bias && res), "dp_gn_mish: FiLM and residual are exclusive");
    if ((int64_t)T * gc <= (int64_t)kGnThreads * kGnRegs)
        gn_mish_kernel<true><<<groups, kGnThreads, 0, st>>>(out, ldo, out2, ldo2, x, ldx, T, gc, scale, bias, eps,
                                                            film_scale, film_bias, res, ldr);
    else
        gn_mish_kernel<false><<<groups, kGnThreads, 0, st>>>(out, ldo, out2, ldo2, x, ldx, T, gc, scale, bias, eps,
                                                             film_scale, film_bias, res, ldr);
    VLA_LAUNCH_CHECK();
}

void launch_spatial_softmax(float* out, const float* x, const float* grid, int npx, int C, hipStream_t st) {
    VLA_REQUIRE(out && x && grid && npx > 0 && C > 0, "spatial_softmax: bad arguments");
    spatial_softmax_kernel<<<(C + 63) / 64, 64, 0, st>>>(out, x, grid, npx, C);
    VLA_LAUNCH_CHECK();
}

void launch_crop_normalize(float* out, const uint8_t* img, int H, int W, int top, int left, int oh, int ow,
                           const float* mean, const float* stdv, float eps, hipStream_t st) {
    VLA_REQUIRE(out && img && oh > 0 && ow > 0 && top >= 0 && left >= 0 && top + oh <= H && left + ow <= W,
                "crop_normalize: crop outside the frame");
    const int64_t n = (int64_t)oh * ow * 3;
    crop_normalize_kernel<<<blocks_for(n), 256, 0, st>>>(out, img, W, top, left, oh, ow, mean, stdv, eps);
    VLA_LAUNCH_CHECK();
}

void launch_dp_gcond(float* g, const float* state, const float* smin, const float* smax, const float* feats,
                     int steps, int sd, int n_cams, int F, float eps, hipStream_t st) {
    const int64_t n = (int64_t)steps * (sd + n_cams * F);
    VLA_REQUIRE(n > 0 && n < INT32_MAX, "dp_gcond: bad shape");
    gcond_kernel<<<blocks_for(n), 256, 0, st>>>(g, state, smin, smax, feats, steps, sd, n_cams, F, eps);
    VLA_LAUNCH_CHECK();
}

void launch_dp_cond_rows(float* gm, const float* temb, const float* gcond, int steps, int D, int G,
                         hipStream_t st) {
    const int64_t n = (int64_t)steps * (D + G);
    VLA_REQUIRE(n > 0, "dp_cond_rows: bad shape");
    cond_rows_kernel<<<blocks_for(n), 256, 0, st>>>(gm, temb, gcond, steps, D, G);
    VLA_LAUNCH_CHECK();
}

void launch_mish(float* x, int64_t n, hipStream_t st) {
    if (n <= 0) return;
    mish_kernel<<<blocks_for(n), 256, 0, st>>>(x, n);
    VLA_LAUNCH_CHECK();
}

void launch_dp_sched_step(float* x, const float* e, const float* z, int n, double sqrt_ap, double sqrt_bp,
                          double c0, double c1, double var, bool ddim, bool clip, double range, hipStream_t st) {
    VLA_REQUIRE(x && e && n > 0 && (ddim || !z || var >= 0.0), "dp_sched_step: bad arguments");
    SchedStep p{sqrt_ap, sqrt_bp, c0, c1, var, -range, range, ddim ? 1 : 0, clip ? 1 : 0, z ? 1 : 0};
    sched_step_kernel<<<blocks_for(n), 256, 0, st>>>(x, e, z, n, p);
    VLA_LAUNCH_CHECK();
}

void launch_dp_actions(float* out, const float* x, int start, int chunk, int A, const float* amin,
                       const float* amax, float eps, bool unnorm, hipStream_t st) {
    VLA_REQUIRE(out && x && chunk > 0 && A > 0 && start >= 0, "dp_actions: bad arguments");
    dp_actions_kernel<<<blocks_for((int64_t)chunk * A), 256, 0, st>>>(out, x, start, chunk, A, amin, amax, eps,
                                                                      unnorm ? 1 : 0);
    VLA_LAUNCH_CHECK();
}

}  // namespace hip
}  // namespace vla
