/*
 * vla_simd_hip.h - C ABI of libvla_simd_hip.so, the MI355X (gfx950) backend of
 * vla.simd's int8 linear + attention hot path.
 *
 * Two layers, as in the reference:
 *   1. the handshake symbols every vla.simd library exports
 *      (include/vla_simd.h:60-62, src/capi_version.cpp:13-15);
 *   2. the op API the reference's src/nn layers call (src/ops/quant_ops.h,
 *      src/ops/lm_ops.h), as extern "C" functions on plain pointers, plus the
 *      device-resident int8 Linear that replaces nn::Linear's int8 state
 *      (src/nn/linear.h:40-48, 85-99).
 *
 * Each op comes in two forms:
 *   vla_<op>(...)        host pointers; copies in, runs on the library's stream,
 *                        copies out, synchronizes. Same argument meaning as the
 *                        reference op of the same name.
 *   vla_<op>_dev(...)    device pointers and a hipStream_t (passed as void*,
 *                        NULL = the null stream); asynchronous, allocates nothing.
 *
 * Layouts (row-major, as src/ops/lm_ops.h:11-14):
 *   activations [seq, K] fp32; quantized activations [seq, ldq] int8 with
 *   ldq >= i8_kpad(K) and columns [K, ldq) zero; int8 weights [N, ldw] int8
 *   (one output channel per row, K contiguous - the GPU layout; the CPU panel
 *   layout of pack_weights_i8 is not used on the device); heads
 *   [seq, n_heads, head_dim].
 *
 * Errors: every fallible call returns vla_status (0 = VLA_OK). HIP runtime
 * failures and C++ exceptions never cross the boundary: they come back as
 * VLA_ERR_EXCEPTION and the message is kept per thread for vla_last_error().
 * Where the reference asserts a precondition (e.g. the int8 K bound,
 * src/nn/linear.cpp:67, tests/test_ops.cpp:79-92) this library returns
 * VLA_ERR_ARG instead of running.
 *
 * Threading: calls on one stream are ordered; the host-pointer forms share one
 * library stream and one grow-only staging arena guarded by a mutex.
 */
#ifndef VLA_SIMD_HIP_H
#define VLA_SIMD_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VLA_API __attribute__((visibility("default")))

#ifndef VLA_ABI_VERSION
#define VLA_ABI_VERSION 1
typedef enum {
    VLA_OK            =  0,
    VLA_ERR_ARG       = -1,
    VLA_ERR_SHAPE     = -2,
    VLA_ERR_EXCEPTION = -3
} vla_status;
#endif

/* Epilogue activation of the int8 linear (applied after dequant + bias). */
typedef enum {
    VLA_ACT_NONE      = 0,
    VLA_ACT_RELU      = 1,  /* relu, src/hal/common/eltwise.cpp:209 */
    VLA_ACT_GELU_TANH = 2,  /* gelu_tanh, eltwise.cpp:74 */
    VLA_ACT_GELU_ERF  = 3   /* gelu_erf, eltwise.cpp:143 */
} vla_act;

/* Attention mask kinds. The reference takes only an additive [seq_q, seq_k]
 * array (src/ops/lm_ops.h:33); the generated kinds produce the same blocked
 * set as the masks its graphs build without reading a [T,T] array. */
typedef enum {
    VLA_MASK_NONE   = 0,  /* gqa_attention_dense semantics */
    VLA_MASK_DENSE  = 1,  /* mask [seq_q, seq_k] additive fp32, lowest()/-inf = blocked */
    VLA_MASK_CAUSAL = 2,  /* key j blocked when j > i + causal_offset */
    VLA_MASK_GROUPS = 3   /* key j blocked when !allow[qg[i]*n_groups + kg[j]] */
} vla_mask_kind;

typedef struct {
    int32_t kind;            /* vla_mask_kind */
    const float* dense;      /* VLA_MASK_DENSE: device or host pointer per call form */
    int32_t causal_offset;   /* VLA_MASK_CAUSAL: usually seq_k - seq_q */
    int32_t n_groups;        /* VLA_MASK_GROUPS: <= 256 */
    const uint8_t* q_group;  /* [seq_q] */
    const uint8_t* k_group;  /* [seq_k] */
    const uint8_t* allow;    /* [n_groups * n_groups], 1 = query group may see key group */
} vla_mask;

/* ---------------------------------------------------------- handshake ---- */

/* include/vla_simd.h:44,60 - returns VLA_ABI_VERSION (1). */
VLA_API int32_t vla_abi_version(void);
/* include/vla_simd.h:61, src/hal/arch.h:54 backend_name() - "hip-gfx950". */
VLA_API const char* vla_backend_name(void);
/* include/vla_simd.h:62, int8_gemm_available() (src/ops/quant_ops.h:41):
 * 1 when a gfx950 device is visible and the int8 kernels can run on it. */
VLA_API int32_t vla_int8_available(void);
/* Message of the last call on this thread that did not return VLA_OK. */
VLA_API const char* vla_last_error(void);

/* ------------------------------------------------ device memory helpers -- */
/* For callers with no allocator of their own (ctypes harnesses, C tests). */
VLA_API int32_t vla_hip_malloc(void** ptr, size_t bytes);
VLA_API int32_t vla_hip_free(void* ptr);
VLA_API int32_t vla_hip_memcpy_h2d(void* dst, const void* src, size_t bytes);
VLA_API int32_t vla_hip_memcpy_d2h(void* dst, const void* src, size_t bytes);
VLA_API int32_t vla_hip_memset(void* dst, int32_t value, size_t bytes);
VLA_API int32_t vla_hip_synchronize(void);
VLA_API int32_t vla_hip_device_name(char* buf, int32_t len);

/* -------------------------------------------- quant_ops.h (int8 linear) -- */

/* i8_kpad (src/ops/quant_ops.h:45, gemm_i8.cpp:30): (K+3) & ~3. */
VLA_API int32_t vla_i8_kpad(int32_t K);

/* quantize_act_i8 (quant_ops.h:76, gemm_i8.cpp:209-244): per row t,
 * s = amax>0 ? max(amax/127, FLT_MIN) : 1, xq = clamp(rne(x/s... as x*(1/s)), +-127),
 * ascale[t] = s. xq is [seq, i8_kpad(K)]; the _dev form takes its stride ldq. */
VLA_API int32_t vla_quantize_act_i8(const float* x, int8_t* xq, float* ascale,
                                    int32_t seq, int32_t K);
VLA_API int32_t vla_quantize_act_i8_dev(const float* x, int8_t* xq, int32_t ldq, float* ascale,
                                        int32_t seq, int32_t K, void* stream);

/* quantize_span_i8 (quant_ops.h:78-80, gemm_i8.cpp:177-207): q[i] =
 * clamp(rne(x[i] * inv), +-127) over n elements with one shared inverse scale
 * (the per-tensor activation quantization of conv2d_i8). */
VLA_API int32_t vla_quantize_span_i8(const float* x, int8_t* q, int64_t n, float inv);
VLA_API int32_t vla_quantize_span_i8_dev(const float* x, int8_t* q, int64_t n, float inv, void* stream);

/* pack_weights_i8 (quant_ops.h:58, gemm_i8.cpp:56-89): the same per-row absmax
 * quantizer over W [N, K] fp32, written as device-layout rows Wq [N, i8_kpad(K)]
 * (no panels, no row sums: the i8 MFMA is signed x signed). */
VLA_API int32_t vla_pack_weights_i8(const float* W, int8_t* Wq, float* wscale,
                                    int32_t N, int32_t K);

/* dense_linear_i8_pre (quant_ops.h:83, reference math gemm_i8.cpp:262-281):
 * out[t,n] = fma((float)acc*wscale[n], ascale[t], bias ? bias[n] : 0) with
 * acc the exact int32 dot of xq row t and Wq row n. xq [seq, i8_kpad(K)],
 * Wq [N, i8_kpad(K)]. bias may be NULL. */
VLA_API int32_t vla_dense_linear_i8_pre(float* out, const int8_t* xq, const float* ascale,
                                        const int8_t* Wq, const float* wscale, const float* bias,
                                        int32_t seq, int32_t N, int32_t K);

/* dense_linear_i8 (quant_ops.h:69, gemm_i8.cpp:246-256): quantize x then the
 * above. The host form allocates its own staging; the _dev form takes the
 * caller-owned scratch the reference takes (quant_ops.h:66-72: xq_scratch
 * holds seq rows of ldq >= i8_kpad(K) bytes, ldq a multiple of 4, and
 * ascale_scratch seq floats), device pointers with row strides (ldx >= K,
 * ldw >= i8_kpad(K), ldo >= N), act / accumulate as in
 * vla_dense_linear_i8_pre_dev, and runs asynchronously on `stream`. */
VLA_API int32_t vla_dense_linear_i8(float* out, const float* x, const int8_t* Wq,
                                    const float* wscale, const float* bias,
                                    int32_t seq, int32_t N, int32_t K);
VLA_API int32_t vla_dense_linear_i8_dev(float* out, int32_t ldo, const float* x, int32_t ldx,
                                        const int8_t* Wq, int32_t ldw, const float* wscale,
                                        const float* bias, int32_t seq, int32_t N, int32_t K,
                                        int8_t* xq_scratch, int32_t ldq, float* ascale_scratch,
                                        int32_t act, int32_t accumulate, void* stream);

/* No counterpart in the reference: vla_dense_linear_i8_dev for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same arguments without the
 * scratch, same values; it allocates nothing. Its scratch is a fixed array in
 * the library's device memory, one per GPU, held until the process ends:
 * 32 MiB of quantized activations (vla_dense_linear_i8_noalloc_max_bytes; the
 * panel layout up to 128 rows, else seq rows of i8_kpad(K) rounded up to 16
 * bytes), 65536 row scales and 8 MiB of split-K partial sums. Larger calls
 * return VLA_ERR_ARG before any launch. Every call on a GPU shares that GPU's
 * array: calls that overlap on one GPU (two streams or threads) race. */
VLA_API int32_t vla_dense_linear_i8_noalloc_dev(float* out, int32_t ldo, const float* x, int32_t ldx,
                                                const int8_t* Wq, int32_t ldw, const float* wscale,
                                                const float* bias, int32_t seq, int32_t N, int32_t K,
                                                int32_t act, int32_t accumulate, void* stream);
VLA_API int64_t vla_dense_linear_i8_noalloc_max_bytes(void);

/* Device form of dense_linear_i8_pre with the fused epilogue options the
 * reference graphs apply right after an int8 forward: act (vla_act, e.g.
 * Linear::forward_gelu, src/nn/linear.cpp:159-168) and accumulate != 0 for
 * out += result (Linear::forward_add, linear.cpp:174-185). ldx/ldw are the
 * int8 row strides (>= i8_kpad(K)), ldo the fp32 output row stride (>= N). */
VLA_API int32_t vla_dense_linear_i8_pre_dev(float* out, int32_t ldo, const int8_t* xq,
                                            int32_t ldx, const float* ascale, const int8_t* Wq,
                                            int32_t ldw, const float* wscale, const float* bias,
                                            int32_t seq, int32_t N, int32_t K, int32_t act,
                                            int32_t accumulate, void* stream);

/* dense_linear_i8_pre_dev with a caller-owned device workspace for split-K
 * (no counterpart in the reference): when the output tiles of a long-K GEMM
 * would leave most CUs idle (more than 128 rows: K >= 1024 on the
 * register-staged tiles; at most 128 rows: K >= 4096 with N/16 column blocks
 * under half the CUs), K is cut into chunks whose int32 partial sums go to
 * `work` and are reduced before the epilogue; the values equal
 * vla_dense_linear_i8_pre_dev's exactly. vla_gemm_i8_split_bytes
 * gives the bytes that shape uses (0: it is not split; at most 8 MiB); a
 * smaller or null workspace just runs unsplit. work: 16-byte aligned. */
VLA_API int64_t vla_gemm_i8_split_bytes(int32_t seq, int32_t N, int32_t K);
VLA_API int32_t vla_dense_linear_i8_pre_split_dev(float* out, int32_t ldo, const int8_t* xq,
                                                  int32_t ldx, const float* ascale,
                                                  const int8_t* Wq, int32_t ldw,
                                                  const float* wscale, const float* bias,
                                                  int32_t seq, int32_t N, int32_t K, int32_t act,
                                                  int32_t accumulate, void* work,
                                                  int64_t work_bytes, void* stream);

/* Panel layout of quantized activations for seq <= 128 rows (the shape of
 * action chunks and decode rows; no counterpart in the reference, whose
 * xq is [seq, i8_kpad(K)]): K is cut into 64-byte panels, each holding all
 * rows' 64 bytes back to back over round_up(seq, 16) rows, so element (t, k)
 * is at byte (k/64) * round_up(seq,16) * 64 + t*64 + k%64; bytes past K in a
 * row's last panel are zero. A 16-row x 64-byte MFMA fragment is then 1 KiB
 * of contiguous memory. vla_i8_panel_bytes gives the buffer size (-1 outside
 * 0..128 rows). The values are exactly those of vla_quantize_act_i8 and
 * vla_dense_linear_i8_pre_dev; only the byte order of xq differs. */
VLA_API int64_t vla_i8_panel_bytes(int32_t seq, int32_t K);
VLA_API int32_t vla_quantize_act_i8_panel_dev(const float* x, int32_t ldx, int8_t* xq,
                                              float* ascale, int32_t seq, int32_t K,
                                              void* stream);
VLA_API int32_t vla_dense_linear_i8_panel_dev(float* out, int32_t ldo, const int8_t* xq,
                                              const float* ascale, const int8_t* Wq,
                                              int32_t ldw, const float* wscale,
                                              const float* bias, int32_t seq, int32_t N,
                                              int32_t K, int32_t act, int32_t accumulate,
                                              void* stream);
/* The same with a split-K workspace, as vla_dense_linear_i8_pre_split_dev
 * (sized by vla_gemm_i8_split_bytes; a smaller or null one runs unsplit). */
VLA_API int32_t vla_dense_linear_i8_panel_split_dev(float* out, int32_t ldo, const int8_t* xq,
                                                    const float* ascale, const int8_t* Wq,
                                                    int32_t ldw, const float* wscale,
                                                    const float* bias, int32_t seq, int32_t N,
                                                    int32_t K, int32_t act, int32_t accumulate,
                                                    void* work, int64_t work_bytes, void* stream);

/* A row op and the int8 quantization of its result in one pass (no
 * counterpart in the reference, which calls rmsnorm or silu_gate and then
 * quantize_act_i8: src/hal/common/norms.cpp:19-35, src/ops/eltwise.cpp:29-64,
 * src/ops/quant_ops.h:17-21): y = op(x) with op 0 identity, 2 RMSNorm with
 * weights w and eps, 3 silu_gate(x, u) (u rows of stride ldu); xq (panel
 * layout, as above) and ascale are what vla_quantize_act_i8_panel_dev gives
 * for y. Rows 16-byte aligned, K a multiple of 4 up to 4096, seq <= 128. */
VLA_API int32_t vla_rowop_quantize_i8_panel_dev(int32_t op, const float* x, int32_t ldx,
                                                const float* u, int32_t ldu, const float* w,
                                                float eps, int8_t* xq, float* ascale,
                                                int32_t seq, int32_t K, void* stream);

/* The same row op fused into the int8 linear that consumes it (no counterpart
 * in the reference; one kernel instead of two): out (+)= exactly what
 * vla_dense_linear_i8_panel_dev gives for the xq / ascale of
 * vla_rowop_quantize_i8_panel_dev. vla_rowop_linear_i8_fits says whether op,
 * seq and K are supported (op 0, 2 or 3; 1 <= seq <= 128; K a multiple of 4
 * up to 2048); out must not overlap x or u; Wq 16-byte aligned with ldw a
 * multiple of 16. */
VLA_API int32_t vla_rowop_linear_i8_fits(int32_t op, int32_t seq, int32_t K);
VLA_API int32_t vla_rowop_linear_i8_dev(float* out, int32_t ldo, int32_t op, const float* x,
                                        int32_t ldx, const float* u, int32_t ldu,
                                        const float* w, float eps, const int8_t* Wq,
                                        int32_t ldw, const float* wscale, const float* bias,
                                        int32_t seq, int32_t N, int32_t K, int32_t act,
                                        int32_t accumulate, void* stream);

/* Exact int32 accumulators acc[t*N+n] (the value gemm_i8.cpp:270-277 forms
 * before its epilogue), for bit-exact parity checks. */
VLA_API int32_t vla_gemm_i8_i32(int32_t* acc, const int8_t* xq, const int8_t* Wq,
                                int32_t seq, int32_t N, int32_t K);
VLA_API int32_t vla_gemm_i8_i32_dev(int32_t* acc, const int8_t* xq, int32_t ldx,
                                    const int8_t* Wq, int32_t ldw, int32_t seq, int32_t N,
                                    int32_t K, void* stream);

/* ------------------------------------ device-resident int8 linear (nn) -- */
/* Replaces nn::Linear's int8 state (src/nn/linear.h:40-48,85-99): the weights
 * are uploaded and quantized once, then live in HBM as int8 rows + per-channel
 * scales + bias. NULL on failure (vla_last_error()); like Linear::init_int8
 * (linear.cpp:66-68) it refuses K > INT_MAX/(255*127). */
typedef struct vla_linear_i8 vla_linear_i8;
/* From fp32 weights W [N,K] (host): quantized on the device with the
 * pack_weights_i8 formula. bias [N] or NULL. */
VLA_API vla_linear_i8* vla_linear_i8_create(const float* W, const float* bias,
                                            int32_t N, int32_t K);
/* From already-quantized weights (host): Wq [N,K] int8 row-major, wscale [N]. */
VLA_API vla_linear_i8* vla_linear_i8_create_q(const int8_t* Wq, const float* wscale,
                                              const float* bias, int32_t N, int32_t K);
VLA_API void vla_linear_i8_free(vla_linear_i8* lin);
/* Device pointers of the resident weights (row stride = vla_linear_i8_ldw). */
VLA_API const int8_t* vla_linear_i8_weights(const vla_linear_i8* lin);
VLA_API const float* vla_linear_i8_wscale(const vla_linear_i8* lin);
VLA_API int32_t vla_linear_i8_ldw(const vla_linear_i8* lin);
/* Linear::forward (linear.cpp:121-133): out [seq,N] = x [seq,K] W^T + bias on
 * the device, quantizing x into the caller's scratch (xq [seq, ldw] int8,
 * ascale [seq]). act / accumulate as in vla_dense_linear_i8_pre_dev. */
VLA_API int32_t vla_linear_i8_forward_dev(const vla_linear_i8* lin, float* out, const float* x,
                                          int32_t seq, int8_t* xq_scratch, float* ascale_scratch,
                                          int32_t act, int32_t accumulate, void* stream);
/* Linear::forward_quantized (linear.cpp:170-172): activations already
 * quantized (xq [seq, ldx]). */
VLA_API int32_t vla_linear_i8_forward_quantized_dev(const vla_linear_i8* lin, float* out,
                                                    const int8_t* xq, int32_t ldx,
                                                    const float* ascale, int32_t seq, int32_t act,
                                                    int32_t accumulate, void* stream);
/* Host copies of the resident state nn::Linear keeps on the host after
 * init_int8 (linear.cpp:97-100): Wq [N, ldq] int8 rows (ldq >= i8_kpad(K),
 * zero past K) and wscale [N]. */
VLA_API int32_t vla_linear_i8_download(const vla_linear_i8* lin, int8_t* Wq, int32_t ldq, float* wscale);
/* Replaces the resident bias with host [N] values (null drops it): the op
 * layer passes nn::Linear's bias per call (linear.cpp:131). */
VLA_API int32_t vla_linear_i8_set_bias(vla_linear_i8* lin, const float* bias);
/* Linear::forward's int8 branch with host pointers over resident weights
 * (linear.cpp:121-133, dense_linear_i8's contract quant_ops.h:66-72): x
 * [seq,K] fp32 in, out [seq,N]; xq_scratch [seq, ldq] (ldq >= i8_kpad(K))
 * and ascale_scratch [seq], each optional, receive the quantized rows. Only
 * activations and outputs cross PCIe. Synchronous. */
VLA_API int32_t vla_linear_i8_forward(const vla_linear_i8* lin, float* out, const float* x, int32_t seq,
                                      int8_t* xq_scratch, int32_t ldq, float* ascale_scratch);
/* Linear::forward_quantized (linear.cpp:170-172) with host pointers over
 * resident weights: xq [seq, ldq] int8 rows (ldq >= i8_kpad(K)), ascale [seq]. */
VLA_API int32_t vla_linear_i8_forward_quantized(const vla_linear_i8* lin, float* out, const int8_t* xq,
                                                int32_t ldq, const float* ascale, int32_t seq);
/* Host-to-device bytes this library has issued since it was loaded, all of
 * them (weights_only 0) or those that carried weights (int8 rows, scales,
 * biases, fp32 weights; weights_only 1). The op API's host forms upload a
 * layer's weights on every call; resident layers once. No counterpart in the
 * reference (its weights are host memory): it shows where PCIe time goes. */
VLA_API int64_t vla_h2d_bytes(int32_t weights_only);

/* ---------------------------------------------------- lm_ops.h (fp32) ---- */

/* gqa_attention_masked (src/ops/lm_ops.h:33-35; semantics of the scalar
 * reference src/hal/scalar/attn.cpp:22-87 and the AVX2 engine
 * src/hal/avx2/attn.cpp:266-447): out = softmax(Q K^T * scale + mask) V per
 * head, kv head = h / (n_q / n_kv); a key with mask == lowest() or score -inf
 * has weight 0; a row with every key blocked is the uniform mean of V.
 * mask [seq_q, seq_k] additive, NULL = dense (gqa_attention_dense,
 * lm_ops.h:43, common/attn.cpp:23-28). head_dim <= 256, head_dim % 4 == 0. */
VLA_API int32_t vla_gqa_attention_masked(float* out, const float* Q, const float* K,
                                         const float* V, int32_t seq_q, int32_t seq_k,
                                         int32_t n_q, int32_t n_kv, int32_t head_dim,
                                         float scale, const float* mask);
VLA_API int32_t vla_gqa_attention_dense(float* out, const float* Q, const float* K,
                                        const float* V, int32_t seq_q, int32_t seq_k,
                                        int32_t n_q, int32_t n_kv, int32_t head_dim, float scale);
/* Device form with explicit row strides (floats between consecutive tokens;
 * 0 = n_heads*head_dim, the lm_ops.h layout) and a mask descriptor whose
 * pointers are device pointers. */
VLA_API int32_t vla_attention_dev(float* out, int32_t ldo, const float* Q, int32_t ldq,
                                  const float* K, int32_t ldk, const float* V, int32_t ldv,
                                  int32_t seq_q, int32_t seq_k, int32_t n_q, int32_t n_kv,
                                  int32_t head_dim, float scale, const vla_mask* mask,
                                  void* stream);
/* Host form of the same, mask pointers on the host (for parity tests). */
VLA_API int32_t vla_attention(float* out, const float* Q, const float* K, const float* V,
                              int32_t seq_q, int32_t seq_k, int32_t n_q, int32_t n_kv,
                              int32_t head_dim, float scale, const vla_mask* mask);

/* layernorm (lm_ops.h:61, src/hal/common/norms.cpp:69-97): per row, mean and
 * variance accumulated in double, out = (float)(x-mean)*inv*w + b; b may be
 * NULL; out may alias x. */
VLA_API int32_t vla_layernorm(float* out, const float* x, const float* w, const float* b,
                              int32_t seq, int32_t hidden, float eps);
VLA_API int32_t vla_layernorm_dev(float* out, const float* x, const float* w, const float* b,
                                  int32_t seq, int32_t hidden, float eps, void* stream);
/* rmsnorm (lm_ops.h:21, norms.cpp:19-35): sum of squares in double. */
VLA_API int32_t vla_rmsnorm(float* out, const float* x, const float* w, int32_t seq,
                            int32_t hidden, float eps);
VLA_API int32_t vla_rmsnorm_dev(float* out, const float* x, const float* w, int32_t seq,
                                int32_t hidden, float eps, void* stream);
/* rope_neox (lm_ops.h:26, norms.cpp:37-67), in place on x [seq, n_heads, head_dim]
 * with row stride ld (0 = n_heads*head_dim). */
VLA_API int32_t vla_rope_neox(float* x, const int32_t* pos, int32_t seq, int32_t n_heads,
                              int32_t head_dim, float base);
VLA_API int32_t vla_rope_neox_dev(float* x, int32_t ld, const int32_t* pos, int32_t seq,
                                  int32_t n_heads, int32_t head_dim, float base, void* stream);

/* Elementwise ops (lm_ops.h:55-73, src/hal/common/eltwise.cpp), in place
 * except silu_gate (out may alias g or u). */
VLA_API int32_t vla_gelu_tanh(float* x, int32_t n);
VLA_API int32_t vla_gelu_erf(float* x, int32_t n);
VLA_API int32_t vla_relu(float* x, int32_t n);
VLA_API int32_t vla_silu_gate(float* out, const float* g, const float* u, int32_t n);
VLA_API int32_t vla_gelu_tanh_dev(float* x, int64_t n, void* stream);
VLA_API int32_t vla_gelu_erf_dev(float* x, int64_t n, void* stream);
VLA_API int32_t vla_relu_dev(float* x, int64_t n, void* stream);
VLA_API int32_t vla_silu_gate_dev(float* out, const float* g, const float* u, int64_t n,
                                  void* stream);
/* out[i] = a[i] + b[i] (residual adds and positional embeddings of the
 * reference graphs, e.g. act_transformer.cpp:227-281). */
VLA_API int32_t vla_add_dev(float* out, const float* a, const float* b, int64_t n, void* stream);

/* dense_linear (lm_ops.h:81-84, src/hal/common/gemm.cpp): the fp32 linear
 * out[t,n] = sum_k x[t,k] W[n,k] + bias[n], W [N,K] row-major, bias may be
 * NULL. fp32 sums in another order than the reference (tolerance class). The
 * graphs use it for the layers their int8 mask leaves in fp32. The _dev form
 * takes row strides, an epilogue act (vla_act, or 4 = silu) and accumulate != 0
 * for out = fmaf(alpha, result, out) (the Euler step x += dt * v of the
 * SmolVLA denoise loop, action_expert.cpp:388). */
VLA_API int32_t vla_dense_linear(float* out, const float* x, const float* W, const float* bias,
                                 int32_t seq, int32_t N, int32_t K);
VLA_API int32_t vla_dense_linear_dev(float* out, int32_t ldo, const float* x, int32_t ldx,
                                     const float* W, int32_t ldw, const float* bias, int32_t seq,
                                     int32_t N, int32_t K, int32_t act, int32_t accumulate,
                                     float alpha, void* stream);

/* ------------------------------------------------------------ convolution -- */
/* W8A8 2-D convolution, tcpu::conv2d_i8 (src/ops/conv_ops.h:31-35,
 * src/hal/common/conv.cpp:424-526): x [H, Wd, Cin] fp32 NHWC -> out
 * [Hout, Wout, Cout], Hout = (H + 2 pad - k) / stride + 1 (square kernel,
 * symmetric zero padding). One activation scale for the whole input tensor,
 * s = max|x| * clip / 127 with clip = TCPU_I8_CLIP (0, 1], default 1, as the
 * reference reads it; weights per output channel over K = k*k*Cin in the patch
 * order [ky][kx][ci] (W [Cout][k][k][Cin] row-major). The values are exactly
 * the reference's. Host form: Wq / wscale as vla_pack_weights_i8 writes them
 * for W viewed as [Cout, K] ([Cout][i8_kpad(K)] rows); any Cout. _dev form:
 * device-resident weights from vla_linear_i8_create(W, bias, Cout, K)
 * (nn::Conv2d::init_int8, src/nn/conv.cpp:50-61), device x / out, and a
 * 256-byte aligned device workspace of vla_conv2d_i8_workspace_bytes (the
 * im2col rows, their scales, the block maxima and the GEMM's split-K sums;
 * the reference's caller-owned xq_scratch); -1 for an invalid shape. */
VLA_API int32_t vla_conv2d_i8(float* out, const float* x, const int8_t* Wq, const float* wscale,
                              const float* bias, int32_t H, int32_t Wd, int32_t Cin, int32_t Cout,
                              int32_t k, int32_t stride, int32_t pad);
/* conv2d_i8 (conv_ops.h:31-35) with host activations over resident weights
 * (vla_linear_i8_create of the [Cout, k*k*Cin] matrix, its bias included):
 * nn::Conv's forward (conv.cpp:55-60) once its weights are on the device.
 * Synchronous. */
VLA_API int32_t vla_conv2d_i8_resident(const vla_linear_i8* lin, float* out, const float* x, int32_t H,
                                       int32_t Wd, int32_t Cin, int32_t k, int32_t stride, int32_t pad);
VLA_API int64_t vla_conv2d_i8_workspace_bytes(int32_t H, int32_t Wd, int32_t Cin, int32_t Cout,
                                              int32_t k, int32_t stride, int32_t pad);
VLA_API int32_t vla_conv2d_i8_dev(const vla_linear_i8* lin, float* out, const float* x, int32_t H,
                                  int32_t Wd, int32_t Cin, int32_t k, int32_t stride, int32_t pad,
                                  void* work, int64_t work_bytes, void* stream);

/* ------------------------------------------------------ checkpoint files -- */
/* The files of a model path, as the policy loaders below read them: a
 * converted directory (<dir>/<name>.meta / .bin), or a vla.simd GGUF that
 * carries them (replaces src/io/files.h:8-17 Mount + InFile with the mount rule
 * of files.cpp find_gguf, and src/io/gguf.cpp + gguf_vla_simd.cpp:29-77 for the
 * format tools/_gguf.py:6-28 writes). A path is a GGUF when it is a *.gguf
 * file, or a directory holding exactly one *.gguf and no *.meta; files the
 * GGUF does not carry are read from disk beside it. vla_ckpt_open returns NULL
 * (vla_last_error()) for a GGUF that is malformed, of another architecture or
 * format version, or names an embedded file outside the model directory.
 * No GPU is used. */
typedef struct vla_ckpt vla_ckpt;
VLA_API vla_ckpt* vla_ckpt_open(const char* path);
VLA_API void vla_ckpt_free(vla_ckpt* c);
/* 1 when the path mounted as a GGUF, 0 for a directory */
VLA_API int32_t vla_ckpt_is_gguf(const vla_ckpt* c);
/* bytes of file `rel` (GGUF, else disk beside it); -1 when there is none */
VLA_API int64_t vla_ckpt_file_size(const vla_ckpt* c, const char* rel);
/* copies file `rel` into buf (cap >= its size); returns a vla_status */
VLA_API int32_t vla_ckpt_read(const vla_ckpt* c, const char* rel, void* buf, int64_t cap);
/* the names of the files the GGUF carries, sorted, '\n'-separated and
 * NUL-terminated into buf when cap is large enough; returns the length
 * needed including the NUL (1 for a directory), or -1 on a null handle */
VLA_API int64_t vla_ckpt_names(const vla_ckpt* c, char* buf, int64_t cap);

/* ------------------------------------------------ device policy graphs ---- */
/* The reference's transformer graphs with every linear, attention, norm and
 * activation on the device and the whole pass replayed as one HIP graph. Each
 * loader reads the reference's own checkpoint files -- from a directory or a
 * vla.simd GGUF, as vla_ckpt_open mounts it (`dir` may name either) -- and
 * takes the int8 mask
 * its model reads from the environment (ACT_INT8 / OCTO_INT8 / SMOLVLA_INT8):
 * the selected layers are quantized once on the device with the
 * pack_weights_i8 formula, the rest stay fp32. NULL on failure
 * (vla_last_error()). One inference per handle at a time
 * (include/vla_simd.h:22-25). Host forms copy in, run and synchronize; _dev
 * forms take device pointers and a hipStream_t (void*, NULL = null stream),
 * run asynchronously and allocate nothing after the first call with a shape. */

/* ACT transformer (ActTransformer, src/models/act/act_transformer.h:36-102):
 * <dir>/act.meta + act.bin as ActTransformer::load (act_transformer.cpp:29-170),
 * img_ch the backbone feature width, int8_mask the ACT_INT8 bits
 * (act_transformer.cpp:27: 1 encoder attention, 2 w1, 4 w2, 8 img_proj,
 * 16 decoder). */
typedef struct vla_act_tf vla_act_tf;
VLA_API vla_act_tf* vla_act_tf_load(const char* dir, int32_t img_ch, int32_t int8_mask);
VLA_API void vla_act_tf_free(vla_act_tf* h);
VLA_API int32_t vla_act_tf_chunk(const vla_act_tf* h);
VLA_API int32_t vla_act_tf_action_dim(const vla_act_tf* h);
VLA_API int32_t vla_act_tf_state_dim(const vla_act_tf* h);
VLA_API int32_t vla_act_tf_dim(const vla_act_tf* h);
/* number of linear layers held as int8 (the count load() prints, :164-167) */
VLA_API int32_t vla_act_tf_int8_layers(const vla_act_tf* h);
/* kernel nodes of the captured graph (0 before the second call with a shape) */
VLA_API int32_t vla_act_tf_graph_nodes(const vla_act_tf* h);
/* ActTransformer::forward (act_transformer.h:98-101, .cpp:358-366) without
 * text tokens: feats [n_cams, fh*fw, img_ch] (the backbone feature maps, NHWC
 * tokens, cameras back to back), state_norm [state_dim] ->
 * actions_norm [chunk, action_dim]. */
VLA_API int32_t vla_act_tf_forward(vla_act_tf* h, const float* feats, int32_t n_cams, int32_t fh,
                                   int32_t fw, const float* state_norm, float* actions_norm);

/* IMPACT's transformer (src/models/impact/impact_model.cpp:59-68,
 * act_transformer.cpp:127-130, 212-250): the same graph loaded with
 * int8_state != 0 (the state projection joins the img_proj int8 group, mask
 * bit 8) and run with a text tail: text / text_pos [n_text_real, dim], of which
 * min(max(n_text_real, 0), act.meta's n_text) rows are appended after the
 * camera tokens (clamp_text). vla_act_tf_forward(_dev) is this with no text. */
VLA_API vla_act_tf* vla_act_tf_load_ex(const char* dir, int32_t img_ch, int32_t int8_mask,
                                       int32_t int8_state);
VLA_API int32_t vla_act_tf_n_text(const vla_act_tf* h);
VLA_API int32_t vla_act_tf_forward_text(vla_act_tf* h, const float* feats, int32_t n_cams, int32_t fh,
                                        int32_t fw, const float* state_norm, const float* text,
                                        const float* text_pos, int32_t n_text_real,
                                        float* actions_norm);
VLA_API int32_t vla_act_tf_forward_text_dev(vla_act_tf* h, const float* feats, int32_t n_cams,
                                            int32_t fh, int32_t fw, const float* state_norm,
                                            const float* text, const float* text_pos,
                                            int32_t n_text_real, float* actions_norm, void* stream);
VLA_API int32_t vla_act_tf_forward_dev(vla_act_tf* h, const float* feats, int32_t n_cams, int32_t fh,
                                       int32_t fw, const float* state_norm, float* actions_norm,
                                       void* stream);

/* Octo block transformer (OctoTransformer, src/models/octo/octo_transformer.h:37-82):
 * <dir>/octo.meta + octo.bin as OctoTransformer::load (octo_transformer.cpp:17-99),
 * int8_mask the OCTO_INT8 bits (octo_model.cpp:60: 1 attention, 2 w1, 4 w2,
 * 8 token projections). An extra meta key "repeat_task 0" drops the per-step
 * copy of the task tokens (the reference always repeats them). */
typedef struct vla_octo_tf vla_octo_tf;
VLA_API vla_octo_tf* vla_octo_tf_load(const char* dir, int32_t int8_mask);
VLA_API void vla_octo_tf_free(vla_octo_tf* h);
VLA_API int32_t vla_octo_tf_dim(const vla_octo_tf* h);
VLA_API int32_t vla_octo_tf_total_tokens(const vla_octo_tf* h, int32_t wnd);
VLA_API int32_t vla_octo_tf_readout_index(const vla_octo_tf* h, int32_t wnd);
/* The checkpoint's shapes the inputs must match: cfg[0..6] = {d, n_task,
 * t5_dim, stem_dim, tok_primary, tok_wrist, max_horizon} (octo.meta keys). */
VLA_API int32_t vla_octo_tf_config(const vla_octo_tf* h, int32_t* cfg);
VLA_API int32_t vla_octo_tf_int8_layers(const vla_octo_tf* h);
VLA_API int32_t vla_octo_tf_graph_nodes(const vla_octo_tf* h);
/* OctoTransformer::forward (octo_transformer.h:75-81, .cpp:144-219):
 * t5_out [n_task, t5_dim], stem_p [wnd, tok_primary, stem_dim], stem_w
 * [wnd, tok_wrist, stem_dim] or NULL, timestep_mask [wnd] (host memory in both
 * forms). out [d] receives the one row the reference writes, out + ro*d with
 * ro = vla_octo_tf_readout_index(wnd): the final-LayerNorm readout token. */
VLA_API int32_t vla_octo_tf_forward(vla_octo_tf* h, const float* t5_out, const float* stem_p,
                                    const float* stem_w, int32_t wnd, const uint8_t* timestep_mask,
                                    float* out);
VLA_API int32_t vla_octo_tf_forward_dev(vla_octo_tf* h, const float* t5_out, const float* stem_p,
                                        const float* stem_w, int32_t wnd, const uint8_t* timestep_mask,
                                        float* out, void* stream);

/* SmolVLA action chunk: the SmolLM2 prefix tower and the action expert
 * (SmollmVlm, src/models/smolvla/smollm2_lm.h:31-47; ActionExpert,
 * action_expert.h:55-93). <dir>/vlm.meta + vlm.bin and aex.meta + aex.bin as
 * their load() (smollm2_lm.cpp:17-83, action_expert.cpp:60-172); int8_mask the
 * SMOLVLA_INT8 bits (smolvla_model.cpp:44: 16 text tower, 32 expert). */
typedef struct vla_smolvla_tf vla_smolvla_tf;
VLA_API vla_smolvla_tf* vla_smolvla_tf_load(const char* dir, int32_t int8_mask);
VLA_API void vla_smolvla_tf_free(vla_smolvla_tf* h);
VLA_API int32_t vla_smolvla_tf_chunk(const vla_smolvla_tf* h);
VLA_API int32_t vla_smolvla_tf_max_action_dim(const vla_smolvla_tf* h);
VLA_API int32_t vla_smolvla_tf_hidden(const vla_smolvla_tf* h);
VLA_API int32_t vla_smolvla_tf_int8_layers(const vla_smolvla_tf* h);
VLA_API int32_t vla_smolvla_tf_graph_nodes(const vla_smolvla_tf* h);
/* SmolvlaModel::predict_normalized after the vision tower and the embedding
 * lookup (smolvla_model.cpp:252-285): prefix [n_prefix, hidden] the assembled
 * prefix embeddings (image and text tokens already scaled by sqrt(hidden),
 * the state token last), pad [n_prefix] (host memory in both forms; 1 real,
 * 0 padding, the last token must be real), noise [chunk, max_action_dim] ->
 * actions [chunk, max_action_dim] (normalized; no RTC guidance). */
VLA_API int32_t vla_smolvla_tf_chunk_run(vla_smolvla_tf* h, const float* prefix, const int32_t* pad,
                                         int32_t n_prefix, const float* noise, float* actions);
VLA_API int32_t vla_smolvla_tf_chunk_dev(vla_smolvla_tf* h, const float* prefix, const int32_t* pad,
                                         int32_t n_prefix, const float* noise, float* actions,
                                         void* stream);


/* SmolVLA's SigLIP vision tower and connector (SiglipVision,
 * src/models/smolvla/siglip_vision.h:23-59): <dir>/vit.meta + vit.bin as
 * SiglipVision::load (siglip_vision.cpp:21-140); int8_mask the vision bits of
 * SMOLVLA_INT8 (smolvla_model.cpp:127-140: 1 attention, 2 w1, 4 w2, 8 patch
 * embedding + modality projection). */
typedef struct vla_siglip_tf vla_siglip_tf;
VLA_API vla_siglip_tf* vla_siglip_tf_load(const char* dir, int32_t int8_mask);
VLA_API void vla_siglip_tf_free(vla_siglip_tf* h);
VLA_API int32_t vla_siglip_tf_img(const vla_siglip_tf* h);
VLA_API int32_t vla_siglip_tf_n_tokens(const vla_siglip_tf* h);
VLA_API int32_t vla_siglip_tf_out_dim(const vla_siglip_tf* h);
VLA_API int32_t vla_siglip_tf_int8_layers(const vla_siglip_tf* h);
VLA_API int32_t vla_siglip_tf_graph_nodes(const vla_siglip_tf* h);
/* SiglipVision::encode (siglip_vision.cpp:151-202): pixels [3, img, img]
 * (CHW, the preprocessed image) -> out [n_tokens, out_dim], the image tokens
 * before SmolvlaModel scales them by sqrt(hidden). The _dev form takes device
 * pointers (16-byte aligned) and a stream and does not synchronize. */
VLA_API int32_t vla_siglip_tf_encode(vla_siglip_tf* h, const float* pixels, float* out);
VLA_API int32_t vla_siglip_tf_encode_dev(vla_siglip_tf* h, const float* pixels, float* out, void* stream);

/* ------------------------------------------------ ACT, model level ------- */

/* The reference's ACT entry points, same names and signatures
 * (include/vla_simd.h:66-81, src/models/act/act_capi.cpp), for callers that
 * bind the model library by name (vla_simd/policy_server.py:203-273 binds
 * vla_act_load / _free / _chunk / _action_dim / _state_dim / _n_cams / _img_h /
 * _img_w / _predict). model_dir holds config.txt, backbone.meta/.bin,
 * act.meta/.bin and stats.bin (tools/convert_act.py's files), or is a vla.simd
 * GGUF carrying them. ACT_INT8 is read at load as act_model.cpp:57-64 reads it
 * (bits 1..16 the transformer's int8 layers, bit 32 the backbone convs from
 * ACT_I8_CONV_FROM to ACT_I8_CONV_TO). predict: images = n_cams uint8 HWC
 * frames at img_h x img_w back to back, state [state_dim] raw, actions
 * [chunk * action_dim] out, un-normalized when unnormalize != 0; the whole
 * pass (normalization, ResNet-18, transformer) runs on the device.
 * Returns VLA_ERR_ARG on a null handle or buffer. */
VLA_API void* vla_act_load(const char* model_dir);
VLA_API void vla_act_free(void* h);
VLA_API int32_t vla_act_chunk(void* h);
VLA_API int32_t vla_act_action_dim(void* h);
VLA_API int32_t vla_act_state_dim(void* h);
VLA_API int32_t vla_act_n_cams(void* h);
VLA_API int32_t vla_act_img_h(void* h);
VLA_API int32_t vla_act_img_w(void* h);
VLA_API int32_t vla_act_predict(void* h, const uint8_t* images, const float* state,
                                int32_t unnormalize, float* actions);
/* Extensions with no counterpart in vla_simd.h: predict on device pointers
 * and a stream (asynchronous: the captured graph reads the frames in place in
 * the stream's order, so they must stay unchanged until the stream has passed
 * the call; other frame pointers than the previous call's start a new
 * capture), the backbone alone (ActModel::encode_view for every camera:
 * feats [n_cams * fh * fw, ch], host pointers, or device pointers and a
 * stream, as predict_dev, the features written in place), its feature grid,
 * and the counts of int8 backbone convs / transformer layers and graph
 * nodes. */
VLA_API int32_t vla_act_predict_dev(void* h, const uint8_t* images, const float* state,
                                    int32_t unnormalize, float* actions, void* stream);
VLA_API int32_t vla_act_encode(void* h, const uint8_t* images, float* feats);
VLA_API int32_t vla_act_encode_dev(void* h, const uint8_t* images, float* feats, void* stream);
VLA_API int32_t vla_act_feat_shape(void* h, int32_t* fh, int32_t* fw, int32_t* ch);
VLA_API int32_t vla_act_int8_convs(void* h);
VLA_API int32_t vla_act_int8_layers(void* h);
VLA_API int32_t vla_act_graph_nodes(void* h);

/* ---------------------------------------------- IMPACT, model level ------- */

/* The reference's IMPACT entry points, same names, signatures and status
 * codes (include/vla_simd.h:206-243, src/models/impact/impact_capi.cpp), for
 * vla_simd/policy_server.py's model-library binding. model_dir holds
 * config.txt (with vocab_full / unk_id), vision.meta/.bin (the trunk with its
 * FiLM points), impact.meta/.bin (the transformer with its text tail),
 * text.meta/.bin (T5-small, the text projection and positions, the FiLM
 * head), vocab.txt, vocab_map.bin and stats.bin, or a vla.simd GGUF carrying
 * them; IMPACT_INT8 (and IMPACT_I8_CONV_FROM / _TO) are read at load.
 * set_instruction runs the language pathway on the device and caches it (a
 * repeated instruction costs nothing); predict sets the instruction, then
 * runs frames [n_cams, img_h, img_w, 3] uint8 and state [state_dim] raw to
 * actions [chunk, action_dim] (un-normalized when unnormalize != 0) on the
 * device. tokens / film copy the current instruction's ids, compacted ids,
 * mask ([n_text] each) and FiLM gamma / beta ([film_total] each) and return
 * the count, VLA_ERR_ARG before any instruction or for a short buffer. */
VLA_API void* vla_impact_load(const char* model_dir);
VLA_API void vla_impact_free(void* h);
VLA_API int32_t vla_impact_chunk(void* h);
VLA_API int32_t vla_impact_action_dim(void* h);
VLA_API int32_t vla_impact_state_dim(void* h);
VLA_API int32_t vla_impact_n_cams(void* h);
VLA_API int32_t vla_impact_img_h(void* h);
VLA_API int32_t vla_impact_img_w(void* h);
VLA_API int32_t vla_impact_n_text(void* h);
VLA_API int32_t vla_impact_set_instruction(void* h, const char* instruction);
VLA_API int32_t vla_impact_predict(void* h, const uint8_t* frames, const float* state, const char* instruction,
                                   int32_t unnormalize, float* actions);
VLA_API int32_t vla_impact_tokens(void* h, int32_t* ids, int32_t* compact, int32_t* mask, int32_t max_elems);
VLA_API int32_t vla_impact_film(void* h, float* gamma, float* beta, int32_t max_elems);
/* Extensions with no counterpart in vla_simd.h: predict on device pointers
 * and a stream (the instruction set first, by set_instruction or predict),
 * and the counts of int8 transformer layers / backbone convs. */
VLA_API int32_t vla_impact_predict_dev(void* h, const uint8_t* frames, const float* state, int32_t unnormalize,
                                       float* actions, void* stream);
VLA_API int32_t vla_impact_int8_layers(void* h);
VLA_API int32_t vla_impact_int8_convs(void* h);

/* ------------------------------------ Diffusion Policy, model level ------- */

/* The reference's Diffusion Policy entry points, same names, signatures and
 * status codes (include/vla_simd.h:245-280,
 * src/models/diffusion/diffusion_capi.cpp): the getters return VLA_ERR_ARG for
 * a null handle. model_dir holds diffusion.meta, rgb_encoder<i>_backbone.meta
 * / .bin and rgb_encoder<i>.bin per encoder, unet.bin and stats.bin, or a
 * vla.simd GGUF carrying them; DIFFUSION_INT8, DP_STEPS and DP_SCHEDULER are
 * read at load. frames [n_obs_steps, n_cams, img_h, img_w, 3] uint8 and state
 * [n_obs_steps, state_dim] are oldest first; noise [1 + num_steps, horizon,
 * action_dim] is the prior then one buffer per DDPM step, or NULL (start from
 * zeros, no noise); actions [chunk, action_dim]. */
VLA_API void* vla_diffusion_load(const char* model_dir);
VLA_API void vla_diffusion_free(void* h);
VLA_API int32_t vla_diffusion_chunk(void* h);
VLA_API int32_t vla_diffusion_horizon(void* h);
VLA_API int32_t vla_diffusion_action_dim(void* h);
VLA_API int32_t vla_diffusion_state_dim(void* h);
VLA_API int32_t vla_diffusion_n_cams(void* h);
VLA_API int32_t vla_diffusion_n_obs_steps(void* h);
VLA_API int32_t vla_diffusion_img_h(void* h);
VLA_API int32_t vla_diffusion_img_w(void* h);
VLA_API int32_t vla_diffusion_num_steps(void* h);
VLA_API int32_t vla_diffusion_is_ddim(void* h);
VLA_API int32_t vla_diffusion_predict(void* h, const uint8_t* frames, const float* state, int32_t unnormalize,
                                      float* actions, const float* noise);
/* Extensions with no counterpart in vla_simd.h: the counts of int8 UNet
 * GEMMs / encoder convs, and the node count of the sampler graph. */
VLA_API int32_t vla_diffusion_int8_layers(void* h);
VLA_API int32_t vla_diffusion_int8_convs(void* h);
VLA_API int32_t vla_diffusion_graph_nodes(void* h);

/* -------------------------------------------- SmolVLA, model level ------- */

/* The reference's SmolVLA entry points, same names and signatures
 * (include/vla_simd.h:83-124, src/models/smolvla/smolvla_capi.cpp), bound by
 * vla_simd/policy_server.py as a model library. load reads the converted
 * directory (or vla.simd GGUF) and the tokenizer's vocab.txt + merges.txt in
 * tok_dir; SMOLVLA_INT8 is read at load (smolvla_model.cpp:44 bits).
 * tokenize: ids / mask [tok_maxlen] as lerobot's tokenizer step produces them
 * (a newline appended, right-padded with pad_token_id / 0, the last
 * tok_maxlen tokens kept); returns the token count, VLA_ERR_ARG on a null
 * argument. predict: n_views native-size uint8 RGB frames [height, width, 3]
 * back to back, the language ids and mask [n_lang] (mask values 0 or 1; the
 * reference adds other values into the positions, the device graph refuses
 * them with VLA_ERR_ARG), state [state_dim] raw, noise [chunk *
 * max_action_dim] or NULL to draw N(0, 1) from mt19937_64(seed), actions
 * [chunk * action_dim] out, un-normalized. VLA_ERR_SHAPE for a view count
 * other than the checkpoint's or a token id outside its vocabulary.
 * predict_rtc adds real-time-chunking guidance: prev [n_prev * action_dim]
 * raw actions of the previous chunk (n_prev <= chunk), weights [chunk], a
 * positive finite max_guidance. Resize, vision tower, prefix and denoise all
 * run on the device. */
VLA_API void* vla_smolvla_load(const char* model_dir, const char* tok_dir);
VLA_API void vla_smolvla_free(void* h);
VLA_API int32_t vla_smolvla_chunk(void* h);
VLA_API int32_t vla_smolvla_action_dim(void* h);
VLA_API int32_t vla_smolvla_state_dim(void* h);
VLA_API int32_t vla_smolvla_n_views(void* h);
VLA_API int32_t vla_smolvla_img_size(void* h);
VLA_API int32_t vla_smolvla_tok_maxlen(void* h);
VLA_API int32_t vla_smolvla_tokenize(void* h, const char* text, int32_t* ids, int32_t* mask);
VLA_API int32_t vla_smolvla_predict(void* h, const uint8_t* frames, int32_t n_views, int32_t height,
                                    int32_t width, const int32_t* lang_tokens, const int32_t* lang_mask,
                                    int32_t n_lang, const float* state, const float* noise, uint64_t seed,
                                    float* actions);
VLA_API int32_t vla_smolvla_predict_rtc(void* h, const uint8_t* frames, int32_t n_views, int32_t height,
                                        int32_t width, const int32_t* lang_tokens, const int32_t* lang_mask,
                                        int32_t n_lang, const float* state, const float* noise, uint64_t seed,
                                        float* actions, const float* prev, int32_t n_prev,
                                        const float* weights, float max_guidance);
/* Extensions with no counterpart in vla_simd.h: the preprocessed views
 * [n_views, 3, img_size, img_size] (resize_with_pad on the device, host
 * pointers), and the counts of int8 layers and graph nodes. */
VLA_API int32_t vla_smolvla_preprocess(void* h, const uint8_t* frames, int32_t n_views, int32_t height,
                                       int32_t width, float* pixels);
VLA_API int32_t vla_smolvla_int8_layers(void* h);
VLA_API int32_t vla_smolvla_graph_nodes(void* h);

/* ----------------------------------------------- Octo, model level ------- */

/* The reference's Octo entry points, same names and signatures
 * (include/vla_simd.h:126-153, src/models/octo/octo_capi.cpp). load reads the
 * converted directory (t5, stem_primary, stem_wrist, octo, head, stats) and
 * the SentencePiece vocab.txt in tok_dir; OCTO_INT8 is read at load
 * (octo_model.cpp:43-58 bits: 1 attention, 2 w1, 4 w2, 8 token projections
 * and stem embeddings, 16 stem convs, 32 the diffusion score net). predict:
 * primary [wnd, 256, 256, 3] and wrist [wnd, 128, 128, 3] (or NULL) uint8,
 * timestep_mask [wnd], the instruction (its T5 embedding is cached), actions
 * [horizon * action_dim] out, un-normalized where the action mask is set when
 * unnormalize != 0. predict_ex takes the DDPM noise [horizon * action_dim] and
 * z [steps * horizon * action_dim], both or neither (VLA_ERR_ARG otherwise);
 * without them they are drawn from mt19937_64(seed). VLA_ERR_SHAPE for wnd
 * outside [1, max_window]. Stems, T5, transformer and head run on the device. */
VLA_API void* vla_octo_load(const char* model_dir, const char* tok_dir);
VLA_API void vla_octo_free(void* h);
VLA_API int32_t vla_octo_horizon(void* h);
VLA_API int32_t vla_octo_action_dim(void* h);
VLA_API int32_t vla_octo_max_window(void* h);
VLA_API int32_t vla_octo_predict(void* h, const uint8_t* primary, const uint8_t* wrist, int32_t wnd,
                                 const uint8_t* timestep_mask, const char* instruction, uint64_t seed,
                                 int32_t unnormalize, float* actions);
VLA_API int32_t vla_octo_predict_ex(void* h, const uint8_t* primary, const uint8_t* wrist, int32_t wnd,
                                    const uint8_t* timestep_mask, const char* instruction, const float* noise,
                                    const float* z, uint64_t seed, int32_t unnormalize, float* actions);
/* Extensions with no counterpart in vla_simd.h: the T5 embedding of an
 * instruction [n_task, t5_dim] (host pointer; n the float count, checked),
 * and the count of int8 layers. */
VLA_API int32_t vla_octo_lang(void* h, const char* instruction, float* out, int64_t n);
VLA_API int32_t vla_octo_int8_layers(void* h);

/* SmolVLA's byte-level BPE tokenizer alone (src/tokenizer/tokenizer.h:16-30,
 * Tokenizer::load + encode), host code that needs no device: tok_dir holds
 * vocab.txt and merges.txt. encode writes at most cap ids and returns the
 * full count (no newline appended, no truncation: vla_smolvla_tokenize adds
 * those). No counterpart in vla_simd.h. */
VLA_API void* vla_bpe_load(const char* tok_dir);
VLA_API void vla_bpe_free(void* h);
VLA_API int32_t vla_bpe_encode(void* h, const char* text, int32_t* ids, int32_t cap);

/* Octo's SentencePiece unigram tokenizer alone (src/tokenizer/
 * t5_tokenizer.h:14-33, T5Tokenizer::load + encode), host code: tok_dir holds
 * vocab.txt ("piece<TAB>score" lines). encode writes exactly max_len ids
 * (pieces cut to max_len - 1, then </s> = 1, then <pad> = 0). No counterpart
 * in vla_simd.h. */
VLA_API void* vla_unigram_load(const char* tok_dir);
VLA_API void vla_unigram_free(void* h);
VLA_API int32_t vla_unigram_encode(void* h, const char* text, int32_t max_len, int32_t* ids);

/* ------------------------------------------------ int8-step probe (tests) -- */

/* Test support with no counterpart in the reference: a record of every int8
 * GEMM one policy-graph pass runs, so a test can check each int8 step on its
 * own against a CPU restatement. While the probe is on (vla_probe_begin until
 * vla_probe_end), the graphs run eagerly (no HIP-graph replay), row ops are
 * not fused into the GEMM (same values), and each int8 GEMM, up to
 * max_records, is copied to the host with a device synchronization per step:
 * the fp32 rows its activations were quantized from (SRC, [M, K]; present
 * when shape[6] = 1), the int8 activations and scales it read (XQ [M, K],
 * ASCALE [M]), its weights (W [N, K] int8, WSCALE [N], BIAS [N] when
 * shape[5] = 1) and its output before and after the launch (BEFORE / AFTER
 * [M, N]). vla_probe_shape writes {M, K, N, act, accumulate, has_bias,
 * has_src}; vla_probe_read copies one field into a host buffer of exactly its
 * size. One probe per process; not for concurrent use. */
enum {
    VLA_PROBE_SRC = 0,
    VLA_PROBE_XQ = 1,
    VLA_PROBE_ASCALE = 2,
    VLA_PROBE_BEFORE = 3,
    VLA_PROBE_AFTER = 4,
    VLA_PROBE_W = 5,
    VLA_PROBE_WSCALE = 6,
    VLA_PROBE_BIAS = 7
};
VLA_API int32_t vla_probe_begin(int32_t max_records);
VLA_API int32_t vla_probe_end(void);
VLA_API int32_t vla_probe_count(void);
VLA_API int32_t vla_probe_shape(int32_t i, int32_t* shape);
VLA_API int32_t vla_probe_read(int32_t i, int32_t what, void* dst, int64_t bytes);

#ifdef __cplusplus
}
#endif
#endif /* VLA_SIMD_HIP_H */
