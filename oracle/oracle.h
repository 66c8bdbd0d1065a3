/*
 * oracle.h - CPU restatement of vla.simd's int8 linear + attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (the HIP library under
 * vla.simd_amd/) links, loads or calls this code. It is used by tests/ as the
 * checker, by __graft_entry__.smoke() to check one GPU call, and by bench.py's
 * cpu_baseline leg. It is plain C99, built by oracle/Makefile into
 * oracle/liboracle.so.
 *
 * Every function names the reference file:line whose arithmetic it restates
 * (paths relative to the vla.simd source tree). Where the reference leaves a
 * rounding choice open (summation order in fp32 attention, the SIMD exp in the
 * softmax) the oracle takes the reference's own scalar form; those results are
 * tolerance-class, the int8 ones are exact.
 *
 * Pinning (what each function is checked against, in tests/test_oracle.py):
 *   orc_quantize_act_i8      golden vectors written by the real reference build
 *                            (tests/golden/), test_ops.cpp:93-112 edge cases,
 *                            brute-force bin check |q*s - x| <= s/2.
 *   orc_gemm_i8_acc          brute-force int64 sum over tiny shapes; golden
 *                            int32 accumulators; linearity in W.
 *   orc_dense_linear_i8_pre  bit-exact vs the reference's dense_linear_i8_ref
 *                            and its AVX-VNNI kernel (golden vectors).
 *   orc_gqa_attention_masked golden vectors (2e-6); double naive softmax
 *                            (test_ops.cpp:161-185); zero mask == no mask;
 *                            fully masked row == uniform mean of V.
 *   orc_layernorm/rmsnorm    golden vectors; double formula (test_ops.cpp:296-321).
 *   orc_gelu_* / silu / relu golden vectors; libm double formula (test_ops.cpp:272-294).
 *   orc_rope_neox            golden vectors from the reference's rope_neox.
 *   orc_conv2d_i8            bit-exact vs the reference's conv2d_i8 built
 *                            from its sources (ref_conv2d_i8), stem / 3x3 /
 *                            1x1-stride-2 / ragged shapes, clip 1 and < 1;
 *                            the im2col against a direct per-tap
 *                            convolution of the quantized input (int64).
 */
#ifndef VLA_ORACLE_H
#define VLA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* K rounded up to a multiple of 4 (src/hal/common/gemm_i8.cpp:30). */
int orc_i8_kpad(int K);

/* test_ops.cpp:31-35 xorshift64 PRNG: fills v[n] with U[lo,hi) draws and
 * advances *state exactly as the reference's frand does. */
void orc_frand_fill(uint64_t* state, float* v, size_t n, float lo, float hi);

/* Per-row symmetric absmax quantization (gemm_i8.cpp:209-244, q8 :49-54,
 * contract src/ops/quant_ops.h:17-21). xq row stride is ldq >= i8_kpad(K);
 * columns [K, ldq) are written as 0. */
void orc_quantize_act_i8(const float* x, int8_t* xq, float* ascale,
                         int seq, int K, int ldq);

/* Weight-side quantizer: same formula per output row (pack_weights_i8,
 * gemm_i8.cpp:56-89), stored row-major [N][ldq] instead of the CPU panels. */
void orc_quantize_weights_i8(const float* W, int8_t* Wq, float* wscale,
                             int N, int K, int ldq);

/* int32 accumulators acc[t*N+n] = sum_k W[n,k]*xq[t,k] (gemm_i8.cpp:270-277).
 * xq [seq][ldx], W [N][ldw], both int8, both zero beyond K. */
void orc_gemm_i8_acc(int32_t* acc, const int8_t* xq, int ldx, const int8_t* Wq, int ldw,
                     int seq, int N, int K);

/* out[t,n] = fma((float)acc*wscale[n], ascale[t], bias ? bias[n] : 0)
 * (gemm_i8.cpp:262-281, the expression at :278). */
void orc_dense_linear_i8_pre(float* out, const int8_t* xq, int ldx, const float* ascale,
                             const int8_t* Wq, int ldw, const float* wscale,
                             const float* bias, int seq, int N, int K);

/* Fused activation applied to an int8 linear's fp32 output the way the
 * reference graphs apply it after forward() (linear.cpp:159-168 for GELU,
 * act_transformer.cpp ReLU). act: 0 none, 1 relu, 2 gelu_tanh, 3 gelu_erf. */
void orc_apply_act(float* x, size_t n, int act);

/* Masked GQA attention, the scalar reference loop (src/hal/scalar/attn.cpp:22-87).
 * mask [seq_q][seq_k] additive or NULL (dense, common/attn.cpp:23-41). A key
 * whose mask entry is -FLT_MAX (lowest()) or whose score is -inf gets weight 0;
 * a row with every key blocked returns the uniform mean of V. */
void orc_gqa_attention_masked(float* out, const float* Q, const float* K, const float* V,
                              int seq_q, int seq_k, int n_q, int n_kv, int head_dim,
                              float scale, const float* mask);

/* src/hal/common/norms.cpp:69-97 (double mean/var, float output). */
void orc_layernorm(float* out, const float* x, const float* w, const float* b,
                   int seq, int hidden, float eps);
/* src/hal/common/norms.cpp:19-35 (double sum of squares). */
void orc_rmsnorm(float* out, const float* x, const float* w, int seq, int hidden, float eps);
/* src/hal/common/norms.cpp:37-67 (double cos/sin tables, NeoX half split). */
void orc_rope_neox(float* x, const int* pos, int seq, int n_heads, int head_dim, float base);

/* src/hal/common/eltwise.cpp scalar forms: gelu_tanh :120-127, gelu_erf
 * :200-206, silu_gate :58-63, relu :209-215. In place except silu_gate. */
void orc_gelu_tanh(float* x, size_t n);
void orc_gelu_erf(float* x, size_t n);
void orc_silu_gate(float* out, const float* g, const float* u, size_t n);
void orc_relu(float* x, size_t n);

float orc_quantize_tensor_i8(const float* x, int8_t* q, size_t n, float clip);
void orc_im2col_i8(int8_t* col, int ldc, const int8_t* xq, int H, int Wd, int Cin, int k, int stride,
                   int pad);
void orc_conv2d_i8(float* out, const float* x, const int8_t* Wq, int ldw, const float* wscale,
                   const float* bias, int H, int Wd, int Cin, int Cout, int k, int stride, int pad,
                   float clip);

#ifdef __cplusplus
}
#endif
#endif /* VLA_ORACLE_H */
