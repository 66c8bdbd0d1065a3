/*
 * ref_shim.cpp - extern "C" wrapper over the REAL vla.simd reference kernels,
 * compiled together with the reference's own hot-path sources (left where they
 * lie under the reference tree; oracle/Makefile names them) into
 * oracle/_ref/libvla_ref.so.
 *
 * TEST INFRASTRUCTURE ONLY: tests/golden/gen_golden.py uses it to write golden
 * vectors, tests/ use it to pin the oracle, and bench.py times it as the CPU
 * baseline ("kind": "reference"). The product never loads it.
 *
 * The only code of this file's own beyond forwarding is the layout transform
 * between row-major int8 weights and the reference's packed panels
 * [N/16][Kp/4][16][4] + int32 row sums (src/ops/quant_ops.h:45-64,
 * src/hal/common/gemm_i8.cpp:56-89): the BASELINE configs hand over int8 weights
 * directly, and the reference kernel only reads its panel format.
 */
#include "hal/arch.h"
#include "ops/lm_ops.h"
#include "ops/conv_ops.h"
#include "ops/quant_ops.h"

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <vector>

#if defined(_OPENMP)
#include <omp.h>
#endif

#define REF_API extern "C" __attribute__((visibility("default")))

REF_API int ref_int8_available(void) { return tcpu::int8_gemm_available() ? 1 : 0; }
REF_API const char* ref_backend_name(void) { return tcpu::hal::backend_name(); }
REF_API int ref_omp_max_threads(void) {
#if defined(_OPENMP)
    return omp_get_max_threads();
#else
    return 1;
#endif
}
REF_API int ref_i8_kpad(int K) { return tcpu::i8_kpad(K); }
REF_API size_t ref_packed_i8_words(int N, int K) { return tcpu::packed_i8_words(N, K); }

REF_API void ref_pack_weights_i8(const float* W, int8_t* Wq, float* wscale, int N, int K) {
    tcpu::pack_weights_i8(W, Wq, wscale, N, K);
}

/* row-major int8 [N][ldw] -> panels + row sums, the layout pack_weights_i8 writes. */
REF_API void ref_panels_from_rows(const int8_t* Wrow, int ldw, int N, int K, int8_t* Wq) {
    const int Kp = tcpu::i8_kpad(K), KG = Kp / 4;
    std::memset(Wq, 0, (size_t)N * Kp);
    int32_t* rowsum = (int32_t*)(Wq + (size_t)N * Kp);
    for (int n = 0; n < N; n++) {
        int32_t sum = 0;
        for (int k = 0; k < K; k++) {
            const int8_t q = Wrow[(size_t)n * ldw + k];
            Wq[((size_t)((n / 16) * KG + k / 4) * 16 + n % 16) * 4 + k % 4] = q;
            sum += q;
        }
        rowsum[n] = sum;
    }
}

/* panels -> row-major int8 [N][ldw] (columns [K, ldw) zeroed). */
REF_API void ref_rows_from_panels(const int8_t* Wq, int N, int K, int8_t* Wrow, int ldw) {
    const int Kp = tcpu::i8_kpad(K), KG = Kp / 4;
    for (int n = 0; n < N; n++) {
        for (int k = 0; k < ldw; k++)
            Wrow[(size_t)n * ldw + k] =
                k < K ? Wq[((size_t)((n / 16) * KG + k / 4) * 16 + n % 16) * 4 + k % 4] : 0;
    }
}

REF_API void ref_quantize_act_i8(const float* x, int8_t* xq, float* ascale, int seq, int K) {
    tcpu::quantize_act_i8(x, xq, ascale, seq, K);
}

REF_API void ref_dense_linear_i8(float* out, const float* x, const int8_t* Wq, const float* wscale,
                                 const float* bias, int seq, int N, int K, int8_t* xq_scratch,
                                 float* ascale_scratch) {
    tcpu::dense_linear_i8(out, x, Wq, wscale, bias, seq, N, K, xq_scratch, ascale_scratch);
}

REF_API void ref_dense_linear_i8_pre(float* out, const int8_t* xq, const float* ascale,
                                     const int8_t* Wq, const float* wscale, const float* bias,
                                     int seq, int N, int K) {
    tcpu::dense_linear_i8_pre(out, xq, ascale, Wq, wscale, bias, seq, N, K);
}

REF_API void ref_dense_linear_i8_ref(float* out, const int8_t* xq, const float* ascale,
                                     const int8_t* Wq, const float* wscale, const float* bias,
                                     int seq, int N, int K) {
    tcpu::dense_linear_i8_ref(out, xq, ascale, Wq, wscale, bias, seq, N, K);
}

REF_API void ref_gqa_attention_masked(float* out, const float* Q, const float* K, const float* V,
                                      int seq_q, int seq_k, int n_q, int n_kv, int head_dim,
                                      float scale, const float* mask) {
    tcpu::gqa_attention_masked(out, Q, K, V, seq_q, seq_k, n_q, n_kv, head_dim, scale, mask);
}

REF_API void ref_gqa_attention_dense(float* out, const float* Q, const float* K, const float* V,
                                     int seq_q, int seq_k, int n_q, int n_kv, int head_dim,
                                     float scale) {
    tcpu::gqa_attention_dense(out, Q, K, V, seq_q, seq_k, n_q, n_kv, head_dim, scale);
}

REF_API void ref_layernorm(float* out, const float* x, const float* w, const float* b, int seq,
                           int hidden, float eps) {
    tcpu::layernorm(out, x, w, b, seq, hidden, eps);
}

REF_API void ref_rmsnorm(float* out, const float* x, const float* w, int seq, int hidden,
                         float eps) {
    tcpu::rmsnorm(out, x, w, seq, hidden, eps);
}

REF_API void ref_rope_neox(float* x, const int* pos, int seq, int n_heads, int head_dim,
                           float base) {
    tcpu::rope_neox(x, pos, seq, n_heads, head_dim, base);
}

/* conv2d_i8 (src/hal/common/conv.cpp:424-526) with weights packed by the
 * reference's pack_weights_i8 over K = k*k*Cin (nn::Conv2d::init_int8,
 * src/nn/conv.cpp:50-61; Cout % 16 == 0). The activation clip is the
 * reference's TCPU_I8_CLIP, read once per process. */
REF_API void ref_conv2d_i8(float* out, const float* x, const float* W, const float* bias, int H, int Wd,
                           int Cin, int Cout, int k, int stride, int pad) {
    const int K = k * k * Cin;
    std::vector<int32_t> packed(tcpu::packed_i8_words(Cout, K));
    std::vector<float> wscale(Cout);
    tcpu::pack_weights_i8(W, reinterpret_cast<int8_t*>(packed.data()), wscale.data(), Cout, K);
    std::vector<int8_t> scratch;
    tcpu::conv2d_i8(out, x, reinterpret_cast<const int8_t*>(packed.data()), wscale.data(), bias, H, Wd, Cin,
                    Cout, k, stride, pad, scratch);
}

/* conv2d_i8 with weights already packed by ref_pack_weights_i8 (the timed
 * CPU baseline: nn::Conv2d::forward's int8 branch, src/nn/conv.cpp:63-69). */
REF_API void ref_conv2d_i8_packed(float* out, const float* x, const int8_t* Wq, const float* wscale,
                                  const float* bias, int H, int Wd, int Cin, int Cout, int k, int stride,
                                  int pad) {
    static thread_local std::vector<int8_t> scratch;
    tcpu::conv2d_i8(out, x, Wq, wscale, bias, H, Wd, Cin, Cout, k, stride, pad, scratch);
}

REF_API void ref_gelu_tanh(float* x, int n) { tcpu::gelu_tanh(x, n); }
REF_API void ref_gelu_erf(float* x, int n) { tcpu::gelu_erf(x, n); }
REF_API void ref_silu_gate(float* out, const float* g, const float* u, int n) {
    tcpu::silu_gate(out, g, u, n);
}
REF_API void ref_relu(float* x, int n) { tcpu::relu(x, n); }

REF_API void ref_dense_linear(float* out, const float* x, const float* W, const float* bias, int seq,
                              int N, int K) {
    tcpu::dense_linear(out, x, W, bias, seq, N, K);
}
