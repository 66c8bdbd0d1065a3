/*
 * oracle.c - CPU restatement of the vla.simd hot path. TEST INFRASTRUCTURE
 * ONLY: see oracle.h for who may call it and what pins each function.
 *
 * Built with -ffp-contract=off so every expression rounds exactly as written:
 * the int8 epilogue below is one explicit fmaf over one rounded product, which
 * is the reference's expression at src/hal/common/gemm_i8.cpp:278 (the AVX2
 * kernel computes the same thing, src/hal/avx2/gemm_i8.cpp:103-104).
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

int orc_i8_kpad(int K) { return (K + 3) & ~3; }

/* tests/test_ops.cpp:31-35 */
void orc_frand_fill(uint64_t* state, float* v, size_t n, float lo, float hi) {
    uint64_t s = *state;
    for (size_t i = 0; i < n; i++) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        v[i] = lo + (hi - lo) * (float)((s >> 40) & 0xFFFFFF) / 16777216.0f;
    }
    *state = s;
}

/* gemm_i8.cpp:49-54: round to nearest even, clamp to the symmetric range. */
static int8_t q8(float v) {
    long r = lrintf(v);
    if (r > 127) r = 127;
    if (r < -127) r = -127;
    return (int8_t)r;
}

/* gemm_i8.cpp:229-243 (scalar body; the AVX2/NEON row quantizers compute the
 * same absmax, the same two IEEE divisions and the same RNE conversion). */
static float row_scale(const float* xt, int K) {
    float amax = 0.0f;
    for (int k = 0; k < K; k++) {
        const float a = fabsf(xt[k]);
        if (a > amax) amax = a;
    }
    if (!(amax > 0.0f)) return 1.0f;
    const float s = amax / 127.0f;
    return s > FLT_MIN ? s : FLT_MIN;
}

static void quantize_row(const float* xt, int8_t* q, float* scale, int K, int ldq) {
    const float s = row_scale(xt, K);
    *scale = s;
    const float inv = 1.0f / s;
    for (int k = 0; k < K; k++) q[k] = q8(xt[k] * inv);
    for (int k = K; k < ldq; k++) q[k] = 0;
}

void orc_quantize_act_i8(const float* x, int8_t* xq, float* ascale, int seq, int K, int ldq) {
    for (int t = 0; t < seq; t++)
        quantize_row(x + (size_t)t * K, xq + (size_t)t * ldq, ascale + t, K, ldq);
}

/* pack_weights_i8 (gemm_i8.cpp:56-89) uses the same per-row formula. */
void orc_quantize_weights_i8(const float* W, int8_t* Wq, float* wscale, int N, int K, int ldq) {
    for (int n = 0; n < N; n++)
        quantize_row(W + (size_t)n * K, Wq + (size_t)n * ldq, wscale + n, K, ldq);
}

/* gemm_i8.cpp:270-277 */
void orc_gemm_i8_acc(int32_t* acc, const int8_t* xq, int ldx, const int8_t* Wq, int ldw,
                     int seq, int N, int K) {
    /* every output is an independent exact integer sum, so threading the
     * (t, n) loop cannot change a value */
#pragma omp parallel for collapse(2) schedule(static)
    for (int t = 0; t < seq; t++) {
        for (int n = 0; n < N; n++) {
            const int8_t* q = xq + (size_t)t * ldx;
            const int8_t* w = Wq + (size_t)n * ldw;
            int32_t a = 0;
            for (int k = 0; k < K; k++) a += (int32_t)w[k] * (int32_t)q[k];
            acc[(size_t)t * N + n] = a;
        }
    }
}

/* gemm_i8.cpp:262-281 */
void orc_dense_linear_i8_pre(float* out, const int8_t* xq, int ldx, const float* ascale,
                             const int8_t* Wq, int ldw, const float* wscale,
                             const float* bias, int seq, int N, int K) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int t = 0; t < seq; t++) {
        for (int n = 0; n < N; n++) {
            const int8_t* q = xq + (size_t)t * ldx;
            const int8_t* w = Wq + (size_t)n * ldw;
            int32_t a = 0;
            for (int k = 0; k < K; k++) a += (int32_t)w[k] * (int32_t)q[k];
            const float p = (float)a * wscale[n];
            out[(size_t)t * N + n] = fmaf(p, ascale[t], bias ? bias[n] : 0.0f);
        }
    }
}

void orc_apply_act(float* x, size_t n, int act) {
    switch (act) {
    case 1: orc_relu(x, n); break;
    case 2: orc_gelu_tanh(x, n); break;
    case 3: orc_gelu_erf(x, n); break;
    default: break;
    }
}

/* src/hal/scalar/attn.cpp:22-87 */
void orc_gqa_attention_masked(float* out, const float* Q, const float* K, const float* V,
                              int seq_q, int seq_k, int n_q, int n_kv, int head_dim,
                              float scale, const float* mask) {
    const int group = n_q / n_kv;
    const float NINF = -INFINITY;
    const float BLOCK = -FLT_MAX;
    float* scores = (float*)malloc(sizeof(float) * (size_t)(seq_k > 0 ? seq_k : 1));
    for (int h = 0; h < n_q; h++) {
        const int kv = h / group;
        for (int t1 = 0; t1 < seq_q; t1++) {
            const float* q = Q + ((size_t)t1 * n_q + h) * head_dim;
            const float* mrow = mask ? mask + (size_t)t1 * seq_k : NULL;
            float maxs = NINF;
            for (int t2 = 0; t2 < seq_k; t2++) {
                if (mrow && mrow[t2] == BLOCK) {
                    scores[t2] = NINF;
                    continue;
                }
                const float* k = K + ((size_t)t2 * n_kv + kv) * head_dim;
                float dot = 0.0f;
                for (int d = 0; d < head_dim; d++) dot += q[d] * k[d];
                dot = dot * scale + (mrow ? mrow[t2] : 0.0f);
                scores[t2] = dot;
                if (dot > maxs) maxs = dot;
            }
            float sum = 0.0f;
            if (maxs == NINF) {
                for (int t2 = 0; t2 < seq_k; t2++) scores[t2] = 1.0f;
                sum = (float)seq_k;
            } else {
                for (int t2 = 0; t2 < seq_k; t2++) {
                    const float s = scores[t2] == NINF ? 0.0f : expf(scores[t2] - maxs);
                    scores[t2] = s;
                    sum += s;
                }
            }
            const float inv = 1.0f / sum;
            float* o = out + ((size_t)t1 * n_q + h) * head_dim;
            for (int d = 0; d < head_dim; d++) o[d] = 0.0f;
            for (int t2 = 0; t2 < seq_k; t2++) {
                if (scores[t2] == 0.0f) continue;
                const float* vv = V + ((size_t)t2 * n_kv + kv) * head_dim;
                const float a = scores[t2] * inv;
                for (int d = 0; d < head_dim; d++) o[d] += a * vv[d];
            }
        }
    }
    free(scores);
}

/* src/hal/common/norms.cpp:69-97 */
void orc_layernorm(float* out, const float* x, const float* w, const float* b,
                   int seq, int hidden, float eps) {
    for (int t = 0; t < seq; t++) {
        const float* xt = x + (size_t)t * hidden;
        float* ot = out + (size_t)t * hidden;
        double mean = 0.0;
        for (int h = 0; h < hidden; h++) mean += xt[h];
        mean /= hidden;
        double var = 0.0;
        for (int h = 0; h < hidden; h++) {
            const double d = xt[h] - mean;
            var += d * d;
        }
        const float inv = (float)(1.0 / sqrt(var / hidden + eps));
        for (int h = 0; h < hidden; h++) {
            const float c = (float)(xt[h] - mean);
            const float y = c * inv * w[h];
            ot[h] = b ? y + b[h] : y;
        }
    }
}

/* src/hal/common/norms.cpp:19-35 */
void orc_rmsnorm(float* out, const float* x, const float* w, int seq, int hidden, float eps) {
    for (int t = 0; t < seq; t++) {
        const float* xt = x + (size_t)t * hidden;
        float* ot = out + (size_t)t * hidden;
        double ss = 0.0;
        for (int h = 0; h < hidden; h++) ss += (double)xt[h] * xt[h];
        const float inv = (float)(1.0 / sqrt(ss / hidden + eps));
        for (int h = 0; h < hidden; h++) ot[h] = xt[h] * inv * w[h];
    }
}

/* src/hal/common/norms.cpp:37-67 */
void orc_rope_neox(float* x, const int* pos, int seq, int n_heads, int head_dim, float base) {
    const int half = head_dim / 2;
    const double theta_scale = pow((double)base, -2.0 / head_dim);
    double* cs = (double*)malloc(sizeof(double) * 2 * (size_t)(half > 0 ? half : 1));
    for (int t = 0; t < seq; t++) {
        double theta = (double)pos[t];
        for (int i = 0; i < half; i++) {
            cs[2 * i] = cos(theta);
            cs[2 * i + 1] = sin(theta);
            theta *= theta_scale;
        }
        for (int hh = 0; hh < n_heads; hh++) {
            float* v = x + ((size_t)t * n_heads + hh) * head_dim;
            for (int i = 0; i < half; i++) {
                const double c = cs[2 * i], s = cs[2 * i + 1];
                const float x0 = v[i], x1 = v[i + half];
                v[i] = (float)(x0 * c - x1 * s);
                v[i + half] = (float)(x0 * s + x1 * c);
            }
        }
    }
    free(cs);
}

/* eltwise.cpp:120-127 */
void orc_gelu_tanh(float* x, size_t n) {
    const float c = 0.7978845608028654f;
    for (size_t i = 0; i < n; i++) {
        const float v = x[i];
        x[i] = 0.5f * v * (1.0f + tanhf(c * (v + 0.044715f * v * v * v)));
    }
}

/* eltwise.cpp:200-206 */
void orc_gelu_erf(float* x, size_t n) {
    const float inv_sqrt2 = 0.70710678118654752f;
    for (size_t i = 0; i < n; i++) {
        const float v = x[i];
        x[i] = 0.5f * v * (1.0f + erff(v * inv_sqrt2));
    }
}

/* eltwise.cpp:58-63 */
void orc_silu_gate(float* out, const float* g, const float* u, size_t n) {
    for (size_t i = 0; i < n; i++) {
        const float v = g[i];
        out[i] = (v / (1.0f + expf(-v))) * u[i];
    }
}

/* eltwise.cpp:209-215 */
void orc_relu(float* x, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (x[i] < 0.0f) x[i] = 0.0f;
}

/* conv2d_i8 (src/hal/common/conv.cpp:424-526, with quantize_tensor_i8 :448-465
 * and im2col_row / im2col_panel :117-176): one scale for the whole NHWC input,
 * s = amax > 0 ? max(amax * clip / 127, FLT_MIN) : 1 (clip = TCPU_I8_CLIP),
 * q = q8(x * (1 / s)) (quantize_span_i8, gemm_i8.cpp:177-206: clamping before
 * or after the rounding gives the same byte); im2col row of output pixel
 * (oy, ox) = taps [ky][kx][ci] at (oy*stride - pad + ky, ox*stride - pad + kx),
 * zero outside the image; then dense_linear_i8_pre with every row scale s.
 * Wq [Cout, ldw] rows over K = k*k*Cin. */
float orc_quantize_tensor_i8(const float* x, int8_t* q, size_t n, float clip) {
    float amax = 0.0f;
    for (size_t i = 0; i < n; i++) {
        const float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    float s = 1.0f;
    if (amax > 0.0f) {
        const float t = amax * clip;
        s = t / 127.0f;
        if (!(s > FLT_MIN)) s = FLT_MIN;
    }
    const float inv = 1.0f / s;
    for (size_t i = 0; i < n; i++) q[i] = q8(x[i] * inv);
    return s;
}

void orc_im2col_i8(int8_t* col, int ldc, const int8_t* xq, int H, int Wd, int Cin, int k, int stride,
                   int pad) {
    const int Hout = (H + 2 * pad - k) / stride + 1, Wout = (Wd + 2 * pad - k) / stride + 1;
    const int K = k * k * Cin;
    for (int oy = 0; oy < Hout; oy++)
        for (int ox = 0; ox < Wout; ox++) {
            int8_t* row = col + ((size_t)oy * Wout + ox) * ldc;
            for (int ky = 0; ky < k; ky++)
                for (int kx = 0; kx < k; kx++)
                    for (int ci = 0; ci < Cin; ci++) {
                        const int iy = oy * stride - pad + ky, ix = ox * stride - pad + kx;
                        const int in = iy >= 0 && iy < H && ix >= 0 && ix < Wd;
                        row[(ky * k + kx) * Cin + ci] = in ? xq[((size_t)iy * Wd + ix) * Cin + ci] : 0;
                    }
            for (int c = K; c < ldc; c++) row[c] = 0;
        }
}

void orc_conv2d_i8(float* out, const float* x, const int8_t* Wq, int ldw, const float* wscale,
                   const float* bias, int H, int Wd, int Cin, int Cout, int k, int stride, int pad,
                   float clip) {
    const int Hout = (H + 2 * pad - k) / stride + 1, Wout = (Wd + 2 * pad - k) / stride + 1;
    const int K = k * k * Cin, Kp = orc_i8_kpad(K), npix = Hout * Wout;
    const size_t nin = (size_t)H * Wd * Cin;
    int8_t* xq = (int8_t*)malloc(nin ? nin : 1);
    int8_t* col = (int8_t*)malloc((size_t)npix * Kp + 1);
    float* as = (float*)malloc(sizeof(float) * (size_t)(npix ? npix : 1));
    const float s = orc_quantize_tensor_i8(x, xq, nin, clip);
    for (int p = 0; p < npix; p++) as[p] = s;
    orc_im2col_i8(col, Kp, xq, H, Wd, Cin, k, stride, pad);
    orc_dense_linear_i8_pre(out, col, Kp, as, Wq, ldw, wscale, bias, npix, Cout, K);
    free(as);
    free(col);
    free(xq);
}
