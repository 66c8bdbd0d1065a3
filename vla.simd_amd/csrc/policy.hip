// policy.hip - the per-query glue of the model-level entry points around the
// transformers: camera preprocessing, token embedding lookup, state and action
// (un)normalization and the flow-matching update with real-time-chunking
// guidance. Each is a single pass over at most a few MB.
#include "act.h"
#include "common.h"
#include "quant_row.h"
#include "wave.h"

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

// dst[t, :] = table[ids[t], :] (fp32), zeros for an id outside [0, vocab)
// (t5_encoder.cpp:96-104)
__global__ __launch_bounds__(256) void embed_f32_kernel(float* __restrict__ dst, const float* __restrict__ table,
                                                        const int32_t* __restrict__ ids, int D, int vocab) {
    const int t = blockIdx.y;
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= D) return;
    const int id = ids[t];
    dst[(int64_t)t * D + j] = id >= 0 && id < vocab ? table[(int64_t)id * D + j] : 0.0f;
}

// SmallStem::encode's input (small_stem.cpp:90-100): [npx, 6] = RGB / 127.5 - 1
// and three goal channels of -1
__global__ __launch_bounds__(256) void stem_input_kernel(float* __restrict__ out, const uint8_t* __restrict__ img,
                                                         int64_t npx) {
    const int64_t n = npx * 6;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t p = i / 6;
        const int c = (int)(i - p * 6);
        out[i] = c < 3 ? (float)img[p * 3 + c] / 127.5f - 1.0f : -1.0f;
    }
}

// GroupNorm (conv.cpp:227-324) with the reference's shifted sums: per channel
// S1 = sum_p (x - K_c), S2 = sum_p (x - K_c)^2 in double, K_c = the first
// pixel's value; per group mean = (sum_c S1_c + n_pixels K_c) / n and
// ss = sum_c S2_c + 2 (K_c - mean) S1_c + n_pixels (K_c - mean)^2, exact
// identities of the two-pass statistics. Three launches, all parallel:
//   groupnorm_partial_kernel   chunk b of the pixels: per-channel (S1, S2)
//                              (coalesced: consecutive threads read
//                              consecutive channels of a pixel);
//   groupnorm_finalize_kernel  per group: the chunks summed in a fixed order,
//                              A = inv * scale, B = bias - mean * inv * scale;
//   groupnorm_apply_kernel     out = x * A[c] + B[c] (+ ReLU).
__global__ __launch_bounds__(256) void groupnorm_partial_kernel(double* __restrict__ part,
                                                                const float* __restrict__ x, int n_pixels, int C,
                                                                int chunk_px) {
    __shared__ double r1[256], r2[256];
    const int t = threadIdx.x;
    const int p0 = blockIdx.x * chunk_px, p1 = p0 + chunk_px < n_pixels ? p0 + chunk_px : n_pixels;
    // C <= 256: lanes pixel lanes of C channels; C > 256: one lane, channels t and t + 256
    const int lanes = C >= 256 ? 1 : 256 / C;
    const int lane = C >= 256 ? 0 : t / C;
    const bool active = lane < lanes;
    for (int cc = 0; cc < C; cc += 256) {
        const int c = C >= 256 ? cc + t : t - lane * C;
        double s1 = 0.0, s2 = 0.0;
        if (active && c < C) {
            const double k = (double)x[c];
            int p = p0 + lane;
            // four pixels' loads in flight, added in pixel order
            for (; p + 3 * lanes < p1; p += 4 * lanes) {
                const float v0 = x[(size_t)p * C + c], v1 = x[(size_t)(p + lanes) * C + c];
                const float v2 = x[(size_t)(p + 2 * lanes) * C + c], v3 = x[(size_t)(p + 3 * lanes) * C + c];
                const double d0 = (double)v0 - k, d1 = (double)v1 - k, d2 = (double)v2 - k, d3 = (double)v3 - k;
                s1 += d0;
                s2 += d0 * d0;
                s1 += d1;
                s2 += d1 * d1;
                s1 += d2;
                s2 += d2 * d2;
                s1 += d3;
                s2 += d3 * d3;
            }
            for (; p < p1; p += lanes) {
                const double d = (double)x[(size_t)p * C + c] - k;
                s1 += d;
                s2 += d * d;
            }
        }
        r1[t] = s1;
        r2[t] = s2;
        __syncthreads();
        // per channel: the lanes in order
        if (C >= 256) {
            if (c < C) {
                part[(size_t)blockIdx.x * 2 * C + c] = r1[t];
                part[(size_t)blockIdx.x * 2 * C + C + c] = r2[t];
            }
        } else if (t < C) {
            double a1 = 0.0, a2 = 0.0;
            for (int l = 0; l < lanes; l++) {
                a1 += r1[l * C + t];
                a2 += r2[l * C + t];
            }
            part[(size_t)blockIdx.x * 2 * C + t] = a1;
            part[(size_t)blockIdx.x * 2 * C + C + t] = a2;
        }
        __syncthreads();
        if (C < 256) break;
    }
}

// one block per group (gc <= 256 channels): lane l of a channel adds chunks
// l, l + lanes, ... in order, the lanes' sums are added in lane order
__global__ __launch_bounds__(256) void groupnorm_finalize_kernel(float* __restrict__ A, float* __restrict__ B,
                                                                 const double* __restrict__ part, int nchunk,
                                                                 const float* __restrict__ x, int n_pixels, int C,
                                                                 int gc, const float* __restrict__ scale,
                                                                 const float* __restrict__ bias, float eps) {
    __shared__ double r1[256], r2[256], S1[256], S2[256], st[2];
    const int t = threadIdx.x, c0 = blockIdx.x * gc;
    const int lanes = 256 / gc, lane = t / gc, cl = t - lane * gc, c = c0 + cl;
    double a1 = 0.0, a2 = 0.0;
    if (lane < lanes) {
        int b = lane;
        for (; b + 3 * lanes < nchunk; b += 4 * lanes) {
            const double u0 = part[(size_t)b * 2 * C + c], u1 = part[(size_t)(b + lanes) * 2 * C + c];
            const double u2 = part[(size_t)(b + 2 * lanes) * 2 * C + c], u3 = part[(size_t)(b + 3 * lanes) * 2 * C + c];
            const double w0 = part[(size_t)b * 2 * C + C + c], w1 = part[(size_t)(b + lanes) * 2 * C + C + c];
            const double w2 = part[(size_t)(b + 2 * lanes) * 2 * C + C + c];
            const double w3 = part[(size_t)(b + 3 * lanes) * 2 * C + C + c];
            a1 += u0;
            a1 += u1;
            a1 += u2;
            a1 += u3;
            a2 += w0;
            a2 += w1;
            a2 += w2;
            a2 += w3;
        }
        for (; b < nchunk; b += lanes) {
            a1 += part[(size_t)b * 2 * C + c];
            a2 += part[(size_t)b * 2 * C + C + c];
        }
    }
    r1[t] = a1;
    r2[t] = a2;
    __syncthreads();
    if (t < gc) {
        double b1 = 0.0, b2 = 0.0;
        for (int l = 0; l < lanes; l++) {
            b1 += r1[l * gc + t];
            b2 += r2[l * gc + t];
        }
        S1[t] = b1;
        S2[t] = b2;
    }
    __syncthreads();
    if (t == 0) {
        const double n = (double)n_pixels * gc;
        double tot = 0.0;
        for (int j = 0; j < gc; j++) tot += S1[j] + (double)n_pixels * (double)x[c0 + j];
        const double mean = tot / n;
        double ss = 0.0;
        for (int j = 0; j < gc; j++) {
            const double dk = (double)x[c0 + j] - mean;
            ss += S2[j] + 2.0 * dk * S1[j] + (double)n_pixels * dk * dk;
        }
        st[0] = mean;
        st[1] = 1.0 / sqrt(ss / n + (double)eps);
    }
    __syncthreads();
    if (t < gc) {
        const double mean = st[0], inv = st[1];
        A[c] = (float)(inv * (double)scale[c]);
        B[c] = (float)fma(-(mean * inv), (double)scale[c], (double)bias[c]);
    }
}

// out = x * A[c] + B[c] (one rounding, as the reference's contracted loop),
// then the fused ReLU (v < 0 -> 0)
__global__ __launch_bounds__(256) void groupnorm_apply_kernel(float* __restrict__ out, const float* __restrict__ x,
                                                              int64_t n, int C, const float* __restrict__ A,
                                                              const float* __restrict__ B, int relu) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int c = (int)(i % C);
        const float v = fmaf(x[i], A[c], B[c]);
        out[i] = relu && v < 0.0f ? 0.0f : v;
    }
}

// the same, 4 channels per thread (C % 4 == 0, 16-byte aligned rows)
__global__ __launch_bounds__(256) void groupnorm_apply4_kernel(float4* __restrict__ out, const float4* __restrict__ x,
                                                               int n4, int C4, const float4* __restrict__ A,
                                                               const float4* __restrict__ B, int relu) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += gridDim.x * blockDim.x) {
        const int c = i % C4;
        const float4 v = x[i], a = A[c], b = B[c];
        float4 o = make_float4(fmaf(v.x, a.x, b.x), fmaf(v.y, a.y, b.y), fmaf(v.z, a.z, b.z), fmaf(v.w, a.w, b.w));
        if (relu) {
            o.x = o.x < 0.0f ? 0.0f : o.x;
            o.y = o.y < 0.0f ? 0.0f : o.y;
            o.z = o.z < 0.0f ? 0.0f : o.z;
            o.w = o.w < 0.0f ? 0.0f : o.w;
        }
        out[i] = o;
    }
}

// DiffusionHead::time_cond's Fourier features for t = 0..steps-1
// (diffusion_head.cpp:129-138): [cos(2 pi t w_i) | sin(2 pi t w_i)]
__global__ __launch_bounds__(256) void fourier_kernel(float* __restrict__ out, const float* __restrict__ w, int steps,
                                                      int TD) {
    const int half = TD / 2;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= steps * half) return;
    const int t = i / half, k = i % half;
    const float f = 6.283185307179586f * (float)t * w[k];
    out[(int64_t)t * TD + k] = cosf(f);
    out[(int64_t)t * TD + half + k] = sinf(f);
}

// in = [a (na) | b (nb) | c (nc)]
__global__ __launch_bounds__(256) void concat3_kernel(float* __restrict__ out, const float* __restrict__ a, int na,
                                                      const float* __restrict__ b, int nb,
                                                      const float* __restrict__ c, int nc) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < na) out[i] = a[i];
    else if (i < na + nb) out[i] = b[i - na];
    else if (i < na + nb + nc) out[i] = c[i - na - nb];
}

// the DDPM update of DiffusionHead::denoise (diffusion_head.cpp:161-177):
// x = clip(a1 * (x - a2 * e) + sb * z, +-max_action)
__global__ __launch_bounds__(256) void ddpm_step_kernel(float* __restrict__ x, const float* __restrict__ e,
                                                        const float* __restrict__ z, int n, float a1, float a2,
                                                        float sb, float max_action) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = fmaf(a1, fmaf(-a2, e[i], x[i]), sb * z[i]);
    x[i] = v < -max_action ? -max_action : v > max_action ? max_action : v;
}


// ------------------------------------------------- Octo's DDPM head, fused --
//
// DiffusionHead::denoise (diffusion_head.cpp:151-177) with DiffusionMlp
// (diffusion.cpp:15-36) for all steps in one workgroup: the head works on one
// row (horizon x action_dim values, hidden H), so each of its ~14 layers per
// step is a few microseconds of launch and latency as a kernel of its own.
// Here the row, the activations and the quantized inputs stay in LDS and the
// weights stream from L2 every step. Each linear repeats the arithmetic of the
// separate kernels: int8 layers quantize their input row as quant_row.h does,
// sum int8 products exactly (any order), then fmaf((float)acc * ws, sa, b);
// fp32 layers sum x * w per output in a fixed order (its own order, fp32
// tolerance); LayerNorm is layernorm_kernel's one-wave double-precision pass.
// Measured on MI355X (Octo-base head, hidden 256, 20 steps): 0.95 ms for the
// whole denoise in one launch, against ~1.0 ms of kernels plus ~280 graph
// nodes layer by layer; about half of it is the barriers and reductions
// between the ~8 dependent layers of a step, half the weight reads of one CU.
// block-wide max; red is free on entry (every phase ends with a barrier)
__device__ __forceinline__ float head_block_max(float v, float* red) {
    v = wave_max_f32(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = 0.0f;
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) m = fmaxf(m, red[w]);
    return m;
}

// y (+)= act(W x + b) for one row; x, y in LDS; q: LDS int8 scratch. The N
// outputs take tpo = 1024 / N threads each (a power of two <= 64, inside one
// wave): thread j of an output walks its weight row's 16-byte chunks j,
// j + tpo, ..., and the tpo partial sums combine through lane exchanges.
__device__ void head_linear(const HeadLin& L, const float* x, float* y, int act, bool acc, int8_t* q, float* red) {
    const int t = threadIdx.x, N = L.N, K = L.K;
    int tpo = 1;
    while (tpo < 64 && tpo * 2 * N <= 1024) tpo *= 2;
    const int n = t / tpo, j = t - n * tpo;
    const bool live = n < N;
    if (L.Wq) {
        // the row quantizer: amax, s = max(amax / 127, FLT_MIN), q = rne(x / s) clamped
        float m = 0.0f;
        for (int k = t; k < K; k += blockDim.x) m = fmaxf(m, fabsf(x[k]));
        const float sa = row_scale(head_block_max(m, red)), inv = 1.0f / sa;
        const int K16 = (K + 15) & ~15;
        for (int k = t; k < K16; k += blockDim.x) q[k] = k < K ? (int8_t)q8(x[k], inv) : (int8_t)0;
        __syncthreads();
        int a = 0;
        if (live) {
            const int8_t* w = L.Wq + (size_t)n * L.ldw;
            for (int c = j * 16; c < K16; c += tpo * 16) {
                const int4 wv = *reinterpret_cast<const int4*>(w + c);
                const int4 qv = *reinterpret_cast<const int4*>(q + c);
                a = __builtin_amdgcn_sdot4(wv.x, qv.x, a, false);
                a = __builtin_amdgcn_sdot4(wv.y, qv.y, a, false);
                a = __builtin_amdgcn_sdot4(wv.z, qv.z, a, false);
                a = __builtin_amdgcn_sdot4(wv.w, qv.w, a, false);
            }
        }
        for (int o = tpo / 2; o > 0; o >>= 1) a += __shfl_xor(a, o, 64);
        if (live && j == 0) {
            float v = fmaf((float)a * L.ws[n], sa, L.b ? L.b[n] : 0.0f);
            if (act == 4) v = act_silu(v);
            y[n] = acc ? y[n] + v : v;
        }
    } else {
        float a = 0.0f;
        if (live) {
            const float* w = L.W + (size_t)n * K;
            for (int k = j; k < K; k += tpo) a = fmaf(x[k], w[k], a);
        }
        // lanes in a fixed pairing order
        for (int o = tpo / 2; o > 0; o >>= 1) a += __shfl_xor(a, o, 64);
        if (live && j == 0) {
            float v = a + (L.b ? L.b[n] : 0.0f);
            if (act == 4) v = act_silu(v);
            y[n] = acc ? fmaf(1.0f, v, y[n]) : v;
        }
    }
    __syncthreads();
}

__global__ __launch_bounds__(1024) void octo_head_kernel(OctoHeadArgs a) {
    extern __shared__ __attribute__((aligned(16))) float hs[];
    const int H = a.H, TD = a.TD, E = a.emb, F = a.flat, IN = TD + E + F;
    const int t = threadIdx.x;
    auto r16 = [](int v) { return (v + 15) & ~15; };
    float* xin = hs;              // [IN]
    float* h = xin + r16(IN);     // [H]
    float* nrm = h + r16(H);      // [H]
    float* wide = nrm + r16(H);   // [4H]
    float* e = wide + r16(4 * H); // [F]
    float* x = e + r16(F);        // [F] the running actions
    float* red = x + r16(F);      // [16]
    int8_t* q = reinterpret_cast<int8_t*>(red + 16);
    for (int i = t; i < F; i += blockDim.x) x[i] = a.noise[i];
    for (int i = t; i < E; i += blockDim.x) xin[TD + i] = a.embv[i];
    __syncthreads();
    for (int s = 0; s < a.steps; s++) {
        const int ts = a.steps - 1 - s;
        for (int i = t; i < TD; i += blockDim.x) xin[i] = a.cond[(size_t)ts * TD + i];
        for (int i = t; i < F; i += blockDim.x) xin[TD + E + i] = x[i];
        __syncthreads();
        head_linear(a.in_proj, xin, h, 0, false, q, red);
        for (int b = 0; b < a.nb; b++) {
            if (t < 64) {  // layernorm_kernel's pass, one wave
                // contracted as eltwise.hip compiles it (the default, fast), so
                // the variance sums round as that kernel's do
#pragma clang fp contract(fast)
                double sum = 0.0;
                for (int k = t; k < H; k += 64) sum += (double)h[k];
                const double mean = wave_sum_f64(sum) / H;
                double v = 0.0;
                for (int k = t; k < H; k += 64) {
                    const double d = (double)h[k] - mean;
                    v += d * d;
                }
                const double var = wave_sum_f64(v);
                const float inv = (float)(1.0 / sqrt(var / H + (double)a.ln_eps));
                for (int k = t; k < H; k += 64) {
                    const float c = (float)((double)h[k] - mean);
                    nrm[k] = a.ln_b[b] ? fmaf(c * inv, a.ln_s[b][k], a.ln_b[b][k]) : c * inv * a.ln_s[b][k];
                }
            }
            __syncthreads();
            head_linear(a.d0[b], nrm, wide, 4, false, q, red);
            head_linear(a.d1[b], wide, h, 0, true, q, red);
        }
        for (int i = t; i < H; i += blockDim.x) h[i] = act_silu(h[i]);
        __syncthreads();
        head_linear(a.out_proj, h, e, 0, false, q, red);
        const float a1 = a.coef[3 * ts], a2 = a.coef[3 * ts + 1], sb = a.coef[3 * ts + 2];
        for (int i = t; i < F; i += blockDim.x) {
            const float v = fmaf(a1, fmaf(-a2, e[i], x[i]), sb * a.z[(size_t)s * F + i]);
            x[i] = v < -a.max_action ? -a.max_action : v > a.max_action ? a.max_action : v;
        }
        __syncthreads();
    }
    for (int i = t; i < F; i += blockDim.x) a.actions[i] = x[i];
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

void launch_embed_f32(float* dst, const float* table, const int32_t* ids, int n, int D, int vocab,
                      hipStream_t st) {
    VLA_REQUIRE(n >= 0 && n < 65536 && D > 0, "embed: bad arguments");
    if (n == 0) return;
    embed_f32_kernel<<<dim3((D + 255) / 256, n), 256, 0, st>>>(dst, table, ids, D, vocab);
    VLA_LAUNCH_CHECK();
}

void launch_stem_input(float* out, const uint8_t* img, int64_t npx, hipStream_t st) {
    VLA_REQUIRE(npx > 0 && out && img, "stem input: bad arguments");
    stem_input_kernel<<<grid_for(npx * 6), 256, 0, st>>>(out, img, npx);
    VLA_LAUNCH_CHECK();
}

namespace {
// pixel chunks of the partial pass: >= 16 pixels each, at most kGnChunks
constexpr int kGnChunks = 256;
int gn_chunk_px(int n_pixels) {
    const int c = (n_pixels + kGnChunks - 1) / kGnChunks;
    return c > 16 ? c : 16;
}
}  // namespace

size_t groupnorm_work_doubles(int n_pixels, int C) {
    const int chunk = gn_chunk_px(n_pixels);
    return (size_t)((n_pixels + chunk - 1) / chunk) * 2 * C;
}

void launch_groupnorm(float* out, const float* x, const float* scale, const float* bias, int n_pixels, int C,
                      int groups, float eps, bool relu, float* A, float* B, double* work, size_t work_doubles,
                      hipStream_t st) {
    VLA_REQUIRE(n_pixels > 0 && C > 0 && groups > 0 && C % groups == 0 && C <= 1024 && C / groups <= 256,
                "groupnorm: bad shape");
    VLA_REQUIRE(work && work_doubles >= groupnorm_work_doubles(n_pixels, C), "groupnorm: workspace too small");
    const int chunk = gn_chunk_px(n_pixels), nchunk = (n_pixels + chunk - 1) / chunk;
    groupnorm_partial_kernel<<<nchunk, 256, 0, st>>>(work, x, n_pixels, C, chunk);
    VLA_LAUNCH_CHECK();
    groupnorm_finalize_kernel<<<groups, 256, 0, st>>>(A, B, work, nchunk, x, n_pixels, C, C / groups, scale, bias,
                                                      eps);
    VLA_LAUNCH_CHECK();
    const int64_t n = (int64_t)n_pixels * C;
    if (C % 4 == 0 && n / 4 < INT32_MAX && (reinterpret_cast<uintptr_t>(out) & 15) == 0 &&
        (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0 &&
        (reinterpret_cast<uintptr_t>(B) & 15) == 0) {
        groupnorm_apply4_kernel<<<grid_for(n / 4), 256, 0, st>>>(
            reinterpret_cast<float4*>(out), reinterpret_cast<const float4*>(x), (int)(n / 4), C / 4,
            reinterpret_cast<const float4*>(A), reinterpret_cast<const float4*>(B), relu ? 1 : 0);
    } else {
        groupnorm_apply_kernel<<<grid_for(n), 256, 0, st>>>(out, x, n, C, A, B, relu ? 1 : 0);
    }
    VLA_LAUNCH_CHECK();
}

void launch_fourier(float* out, const float* w, int steps, int TD, hipStream_t st) {
    VLA_REQUIRE(steps > 0 && TD > 0 && TD % 2 == 0, "fourier: bad shape");
    const int n = steps * (TD / 2);
    fourier_kernel<<<(n + 255) / 256, 256, 0, st>>>(out, w, steps, TD);
    VLA_LAUNCH_CHECK();
}

void launch_concat3(float* out, const float* a, int na, const float* b, int nb, const float* c, int nc,
                    hipStream_t st) {
    const int n = na + nb + nc;
    concat3_kernel<<<(n + 255) / 256, 256, 0, st>>>(out, a, na, b, nb, c, nc);
    VLA_LAUNCH_CHECK();
}

size_t octo_head_lds_bytes(int H, int TD, int emb, int flat) {
    auto r16 = [](size_t v) { return (v + 15) & ~(size_t)15; };
    const size_t IN = (size_t)TD + emb + flat;
    const size_t floats = r16(IN) + 2 * r16(H) + r16(4 * (size_t)H) + 2 * r16(flat) + 16;
    const size_t qbytes = r16(IN > 4 * (size_t)H ? IN : 4 * (size_t)H);
    return floats * 4 + qbytes;
}

// head_linear computes outputs n < 1024 / tpo with tpo >= 1, reads K inputs
// from an LDS row sized for its layer, and (int8) 16-byte weight chunks up to
// round16(K)
static bool head_lin_fits(const HeadLin& L, int K, int max_n) {
    if (L.K != K || L.N < 1 || L.N > max_n || L.N > 1024) return false;
    if (L.Wq) return L.ws && L.ldw >= ((K + 15) & ~15) && L.ldw % 16 == 0;
    return L.W != nullptr;
}

void launch_octo_head(const OctoHeadArgs& a, hipStream_t st) {
    const size_t lds = octo_head_lds_bytes(a.H, a.TD, a.emb, a.flat);
    VLA_REQUIRE(a.nb >= 0 && a.nb <= kOctoHeadMaxBlocks && lds <= 64 * 1024 && a.steps > 0,
                "octo head: shape beyond the fused kernel");
    VLA_REQUIRE(a.H > 0 && 4 * a.H <= 1024 && a.flat > 0 && a.flat <= 1024 && a.TD >= 0 && a.emb >= 0,
                "octo head: hidden width (x4) and action row must be at most 1024");
    bool fits = head_lin_fits(a.in_proj, a.TD + a.emb + a.flat, a.H) && a.in_proj.N == a.H &&
                head_lin_fits(a.out_proj, a.H, a.flat) && a.out_proj.N == a.flat;
    for (int b = 0; b < a.nb && fits; b++)
        fits = a.ln_s[b] && head_lin_fits(a.d0[b], a.H, 4 * a.H) && head_lin_fits(a.d1[b], a.d0[b].N, a.H) &&
               a.d1[b].N == a.H;
    VLA_REQUIRE(fits, "octo head: a layer's width does not match the fused kernel's rows (N <= 1024)");
    octo_head_kernel<<<1, 1024, lds, st>>>(a);
    VLA_LAUNCH_CHECK();
}

void launch_ddpm_step(float* x, const float* e, const float* z, int n, float a1, float a2, float sb,
                      float max_action, hipStream_t st) {
    ddpm_step_kernel<<<(n + 255) / 256, 256, 0, st>>>(x, e, z, n, a1, a2, sb, max_action);
    VLA_LAUNCH_CHECK();
}

void launch_rtc_step(float* x, const float* v, const float* prev, const float* weights, const float* gw, int step,
                     int rows, int cols, float time, float dt, hipStream_t st) {
    rtc_step_kernel<<<grid_for((int64_t)rows * cols), 256, 0, st>>>(x, v, prev, weights, gw, step, rows, cols, time,
                                                                    dt);
    VLA_LAUNCH_CHECK();
}

// One thread per column: the live rows summed in row order, then scaled by
// 1 / live, the float operations of the host loop (t5_text.cpp:115-128).
__global__ __launch_bounds__(256) void masked_row_mean_kernel(float* __restrict__ out, const float* __restrict__ x,
                                                              int ldx, const int32_t* __restrict__ mask, int rows,
                                                              int D) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= D) return;
    float acc = 0.0f;
    int live = 0;
    for (int t = 0; t < rows; t++) {
        if (!mask[t]) continue;
        acc += x[(size_t)t * ldx + i];
        live++;
    }
    if (live > 0) acc *= 1.0f / (float)live;
    out[i] = acc;
}

void launch_masked_row_mean(float* out, const float* x, int ldx, const int32_t* mask, int rows, int D,
                            hipStream_t st) {
    VLA_REQUIRE(out && x && mask && rows > 0 && D > 0 && ldx >= D, "masked_row_mean: bad arguments");
    masked_row_mean_kernel<<<(D + 255) / 256, 256, 0, st>>>(out, x, ldx, mask, rows, D);
    VLA_LAUNCH_CHECK();
}

}  // namespace hip
}  // namespace vla
