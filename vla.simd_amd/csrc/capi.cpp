// capi.cpp - the extern "C" surface declared in include/vla_simd_hip.h.
//
// Host-pointer forms: lock the staging arena, upload, run on the library
// stream, download, synchronize. Device forms: validate and launch on the
// caller's stream. Every entry goes through guarded(), so HIP failures and
// C++ exceptions come back as vla_status codes (include/vla_simd.h:15-20).

#include "vla_simd_hip.h"

#include "linear.h"
#include "runtime.h"

#include <cstdlib>

using namespace vla::hip;

namespace {

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

AttnArgs make_attn(float* out, int ldo, const float* Q, int ldq, const float* K, int ldk,
                   const float* V, int ldv, int sq, int sk, int nq, int nkv, int hd, float scale,
                   const vla_mask* mask) {
    AttnArgs a{};
    a.out = out;
    a.ldo = ldo ? ldo : nq * hd;
    a.Q = Q;
    a.ldq = ldq ? ldq : nq * hd;
    a.K = K;
    a.ldk = ldk ? ldk : nkv * hd;
    a.V = V;
    a.ldv = ldv ? ldv : nkv * hd;
    a.seq_q = sq;
    a.seq_k = sk;
    a.n_q = nq;
    a.n_kv = nkv;
    a.head_dim = hd;
    a.scale = scale;
    a.mask_kind = mask ? mask->kind : VLA_MASK_NONE;
    if (mask) {
        a.mask = mask->dense;
        a.ldm = sk;
        a.causal_offset = mask->causal_offset;
        a.n_groups = mask->n_groups;
        a.q_group = mask->q_group;
        a.k_group = mask->k_group;
        a.allow = mask->allow;
    }
    return a;
}

}  // namespace

extern "C" {

// ------------------------------------------------------------- handshake --

VLA_API int32_t vla_abi_version(void) { return VLA_ABI_VERSION; }
VLA_API const char* vla_backend_name(void) { return "hip-gfx950"; }
VLA_API int32_t vla_int8_available(void) { return device_is_gfx950() ? 1 : 0; }
VLA_API const char* vla_last_error(void) { return last_error(); }

// ------------------------------------------------------- memory helpers --

VLA_API int32_t vla_hip_malloc(void** ptr, size_t bytes) {
    return guarded("vla_hip_malloc", [&] {
        VLA_REQUIRE(ptr, "null output pointer");
        *ptr = nullptr;
        VLA_HIP_CHECK(hipMalloc(ptr, bytes ? bytes : 1));
    });
}
VLA_API int32_t vla_hip_free(void* ptr) {
    return guarded("vla_hip_free", [&] {
        if (ptr) VLA_HIP_CHECK(hipFree(ptr));
    });
}
VLA_API int32_t vla_hip_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    return guarded("vla_hip_memcpy_h2d", [&] { VLA_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice)); });
}
VLA_API int32_t vla_hip_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    return guarded("vla_hip_memcpy_d2h", [&] { VLA_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost)); });
}
VLA_API int32_t vla_hip_memset(void* dst, int32_t value, size_t bytes) {
    return guarded("vla_hip_memset", [&] {
        VLA_HIP_CHECK(hipMemset(dst, value, bytes));
        VLA_HIP_CHECK(hipStreamSynchronize(nullptr));  // done before the caller's other streams use dst
    });
}
VLA_API int32_t vla_hip_synchronize(void) {
    return guarded("vla_hip_synchronize", [&] { VLA_HIP_CHECK(hipDeviceSynchronize()); });
}
VLA_API int32_t vla_hip_device_name(char* buf, int32_t len) {
    return guarded("vla_hip_device_name", [&] {
        VLA_REQUIRE(buf && len > 0, "null buffer");
        int dev = 0;
        VLA_HIP_CHECK(hipGetDevice(&dev));
        hipDeviceProp_t p;
        VLA_HIP_CHECK(hipGetDeviceProperties(&p, dev));
        std::snprintf(buf, (size_t)len, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
    });
}

// ------------------------------------------------------------ quant ops --

VLA_API int32_t vla_i8_kpad(int32_t K) { return kpad4(K); }

static int32_t quantize_host(const char* where, const float* x, int8_t* xq, float* ascale,
                             int32_t seq, int32_t K) {
    return guarded(where, [&] {
        VLA_REQUIRE(seq >= 0 && K > 0, "need seq >= 0 and K > 0");
        VLA_REQUIRE(seq == 0 || (x && xq && ascale), "null buffer");
        if (seq == 0) return;
        const int Kp = kpad4(K);
        Staging& S = staging();
        auto lk = S.lock();
        hipStream_t st = library_stream();
        S.reset(align256((size_t)seq * K * 4) + align256((size_t)seq * Kp) + align256((size_t)seq * 4));
        const float* dx = S.upload(x, (size_t)seq * K, st);
        int8_t* dq = S.alloc<int8_t>((size_t)seq * Kp);
        float* ds = S.alloc<float>(seq);
        launch_quantize_rows(dx, K, dq, Kp, ds, seq, K, st);
        VLA_HIP_CHECK(hipMemcpyAsync(xq, dq, (size_t)seq * Kp, hipMemcpyDeviceToHost, st));
        VLA_HIP_CHECK(hipMemcpyAsync(ascale, ds, (size_t)seq * 4, hipMemcpyDeviceToHost, st));
        VLA_HIP_CHECK(hipStreamSynchronize(st));
    });
}

VLA_API int32_t vla_quantize_act_i8(const float* x, int8_t* xq, float* ascale, int32_t seq,
                                    int32_t K) {
    return quantize_host("vla_quantize_act_i8", x, xq, ascale, seq, K);
}

VLA_API int32_t vla_quantize_act_i8_dev(const float* x, int8_t* xq, int32_t ldq, float* ascale,
                                        int32_t seq, int32_t K, void* stream) {
    return guarded("vla_quantize_act_i8_dev", [&] {
        launch_quantize_rows(x, K, xq, ldq, ascale, seq, K, as_stream(stream));
    });
}

VLA_API int32_t vla_quantize_span_i8_dev(const float* x, int8_t* q, int64_t n, float inv, void* stream) {
    return guarded("vla_quantize_span_i8_dev", [&] { launch_quantize_span(x, q, n, inv, as_stream(stream)); });
}

VLA_API int32_t vla_quantize_span_i8(const float* x, int8_t* q, int64_t n, float inv) {
    return guarded("vla_quantize_span_i8", [&] {
        VLA_REQUIRE(n >= 0 && (n == 0 || (x && q)), "need n >= 0 and non-null buffers");
        if (n == 0) return;
        Staging& S = staging();
        auto lk = S.lock();
        hipStream_t st = library_stream();
        S.reset(align256((size_t)n * 4) + align256((size_t)n));
        const float* dx = S.upload(x, (size_t)n, st);
        int8_t* dq = S.alloc<int8_t>((size_t)n);
        launch_quantize_span(dx, dq, n, inv, st);
        VLA_HIP_CHECK(hipMemcpyAsync(q, dq, (size_t)n, hipMemcpyDeviceToHost, st));
        VLA_HIP_CHECK(hipStreamSynchronize(st));
    });
}

VLA_API int32_t vla_pack_weights_i8(const float* W, int8_t* Wq, float* wscale, int32_t N,
                                    int32_t K) {
    // pack_weights_i8 (gemm_i8.cpp:56-89) is the same per-row quantizer over W.
    return quantize_host("vla_pack_weights_i8", W, Wq, wscale, N, K);
}

static void gemm_host(float* out, int32_t* acc32, const int8_t* xq, const float* ascale,
                      const int8_t* Wq, const float* wscale, const float* bias, int seq, int N, int K) {
    VLA_REQUIRE(seq >= 0 && N > 0 && K > 0, "need seq >= 0, N > 0, K > 0");
    VLA_REQUIRE(K <= kMaxI8K, "K exceeds the int8 accumulator bound INT_MAX/(255*127)");
    VLA_REQUIRE(seq == 0 || (xq && Wq && (acc32 || (out && ascale && wscale))), "null buffer");
    if (seq == 0) return;
    const int Kp = kpad4(K);
    Staging& S = staging();
    auto lk = S.lock();
    hipStream_t st = library_stream();
    S.reset(align256((size_t)seq * Kp) + align256((size_t)N * Kp) + align256((size_t)seq * 4) +
            2 * align256((size_t)N * 4) + align256((size_t)seq * N * 4));
    GemmArgs a{};
    a.A = S.upload(xq, (size_t)seq * Kp, st);
    a.lda = Kp;
    a.B = S.upload(Wq, (size_t)N * Kp, st, true);
    a.ldb = Kp;
    a.ascale = S.upload(ascale, (size_t)seq, st);
    a.wscale = S.upload(wscale, (size_t)N, st, true);
    a.bias = S.upload(bias, (size_t)N, st, true);
    void* dout = S.take((size_t)seq * N * 4);
    if (acc32) a.acc32 = static_cast<int32_t*>(dout);
    else a.out = static_cast<float*>(dout);
    a.ldo = N;
    a.M = seq;
    a.N = N;
    a.K = K;
    launch_gemm_i8(a, st);
    VLA_HIP_CHECK(hipMemcpyAsync(acc32 ? (void*)acc32 : (void*)out, dout, (size_t)seq * N * 4,
                                 hipMemcpyDeviceToHost, st));
    VLA_HIP_CHECK(hipStreamSynchronize(st));
}

VLA_API int32_t vla_dense_linear_i8_pre(float* out, const int8_t* xq, const float* ascale,
                                        const int8_t* Wq, const float* wscale, const float* bias,
                                        int32_t seq, int32_t N, int32_t K) {
    return guarded("vla_dense_linear_i8_pre", [&] {
        gemm_host(out, nullptr, xq, ascale, Wq, wscale, bias, seq, N, K);
    });
}

VLA_API int32_t vla_gemm_i8_i32(int32_t* acc, const int8_t* xq, const int8_t* Wq, int32_t seq,
                                int32_t N, int32_t K) {
    return guarded("vla_gemm_i8_i32", [&] {
        VLA_REQUIRE(acc, "null output");
        gemm_host(nullptr, acc, xq, nullptr, Wq, nullptr, nullptr, seq, N, K);
    });
}

VLA_API int32_t vla_dense_linear_i8(float* out, const float* x, const int8_t* Wq,
                                    const float* wscale, const float* bias, int32_t seq, int32_t N,
                                    int32_t K) {
    return guarded("vla_dense_linear_i8", [&] {
        VLA_REQUIRE(seq >= 0 && N > 0 && K > 0, "need seq >= 0, N > 0, K > 0");
        VLA_REQUIRE(K <= kMaxI8K, "K exceeds the int8 accumulator bound INT_MAX/(255*127)");
        VLA_REQUIRE(seq == 0 || (out && x && Wq && wscale), "null buffer");
        if (seq == 0) return;
        const int Kp = kpad4(K);
        Staging& S = staging();
        auto lk = S.lock();
        hipStream_t st = library_stream();
        S.reset(align256((size_t)seq * K * 4) + align256((size_t)seq * Kp) + align256((size_t)N * Kp) +
                align256((size_t)seq * 4) + 2 * align256((size_t)N * 4) + align256((size_t)seq * N * 4));
        const float* dx = S.upload(x, (size_t)seq * K, st);
        int8_t* dq = S.alloc<int8_t>((size_t)seq * Kp);
        float* ds = S.alloc<float>(seq);
        launch_quantize_rows(dx, K, dq, Kp, ds, seq, K, st);
        GemmArgs a{};
        a.A = dq;
        a.lda = Kp;
        a.B = S.upload(Wq, (size_t)N * Kp, st, true);
        a.ldb = Kp;
        a.ascale = ds;
        a.wscale = S.upload(wscale, (size_t)N, st, true);
        a.bias = S.upload(bias, (size_t)N, st, true);
        a.out = S.alloc<float>((size_t)seq * N);
        a.ldo = N;
        a.M = seq;
        a.N = N;
        a.K = K;
        launch_gemm_i8(a, st);
        VLA_HIP_CHECK(hipMemcpyAsync(out, a.out, (size_t)seq * N * 4, hipMemcpyDeviceToHost, st));
        VLA_HIP_CHECK(hipStreamSynchronize(st));
    });
}

static RowQArgs rowop_args(int32_t op, const float* x, int32_t ldx, const float* u, int32_t ldu,
                           const float* w, float eps, int32_t seq, int32_t K);

// Up to 16 rows of the op API take the fused row-op GEMM (the quantization
// inside the GEMM) where it applies. Graph replays on MI355X, quantize + GEMM
// -> fused: 1x512x3200 5.22 -> 3.36 us, 1x960x2560 5.70 -> 4.02, 1x768x3072
// 5.60 -> 3.85, 16x512x3200 5.48 -> 3.92, 16x960x2560 5.99 -> 4.83,
// 16x768x3072 5.88 -> 4.52; from 50 rows on it was slower (50x960x2560 7.00
// -> 8.56, 100x960x2560 8.3 -> 14.6). VLA_HIP_OP_FUSE=0 keeps the two
// launches (A/B runs; outputs and scratch bytes are the same either way).
static bool op_fuses(const float* x, int ldx, const int8_t* Wq, int ldw, const float* out, int ldo,
                     const int8_t* xq, int ldq, const float* ascale, int seq, int N, int K) {
    const char* e = std::getenv("VLA_HIP_OP_FUSE");
    if (e && std::atoi(e) == 0) return false;
    if (seq < 1 || seq > 16 || !rowop_gemm_fits(0, seq, K)) return false;
    if (ldx < K || ldx % 4 || !aligned(x, 16) || ldw < kpad4(K) || ldw % 16 || !aligned(Wq, 16)) return false;
    if (ldq < kpad4(K) || ldq % 4 || !aligned(xq, 4) || !ascale || ldo < N) return false;
    const uintptr_t o0 = (uintptr_t)out, o1 = o0 + ((size_t)(seq - 1) * ldo + N) * sizeof(float);
    const uintptr_t x0 = (uintptr_t)x, x1 = x0 + ((size_t)(seq - 1) * ldx + K) * sizeof(float);
    return o1 <= x0 || x1 <= o0;  // out apart from the rows read (else the two launches)
}

VLA_API int32_t vla_dense_linear_i8_dev(float* out, int32_t ldo, const float* x, int32_t ldx,
                                        const int8_t* Wq, int32_t ldw, const float* wscale,
                                        const float* bias, int32_t seq, int32_t N, int32_t K,
                                        int8_t* xq_scratch, int32_t ldq, float* ascale_scratch,
                                        int32_t act, int32_t accumulate, void* stream) {
    return guarded("vla_dense_linear_i8_dev", [&] {
        VLA_REQUIRE(seq >= 0 && N > 0 && K > 0, "need seq >= 0, N > 0, K > 0");
        VLA_REQUIRE(K <= kMaxI8K, "K exceeds the int8 accumulator bound INT_MAX/(255*127)");
        VLA_REQUIRE(seq == 0 || (out && x && Wq && wscale && xq_scratch && ascale_scratch), "null buffer");
        if (seq == 0) return;
        hipStream_t st = as_stream(stream);
        // the reference's contract: xq_scratch holds seq x i8_kpad(K) bytes
        // (here with row stride ldq), ascale_scratch seq floats
        if (op_fuses(x, ldx, Wq, ldw, out, ldo, xq_scratch, ldq, ascale_scratch, seq, N, K)) {
            // a few rows: quantized inside the GEMM (every block repeats the
            // cheap row work instead of waiting for a separate launch), the
            // scratch filled by the same kernel with the same bytes
            RowQArgs r = rowop_args(0, x, ldx, nullptr, 0, nullptr, 0.0f, seq, K);
            r.q = xq_scratch;
            r.ldq = ldq;
            r.qs = ascale_scratch;
            GemmArgs a{};
            a.B = Wq;
            a.ldb = ldw;
            a.wscale = wscale;
            a.bias = bias;
            a.out = out;
            a.ldo = ldo;
            a.M = seq;
            a.N = N;
            a.K = K;
            a.act = act;
            a.accumulate = accumulate;
            launch_gemm_i8_rowop(r, a, st);
            return;
        }
        launch_quantize_rows(x, ldx, xq_scratch, ldq, ascale_scratch, seq, K, st);
        GemmArgs a{};
        a.A = xq_scratch;
        a.lda = ldq;
        a.B = Wq;
        a.ldb = ldw;
        a.ascale = ascale_scratch;
        a.wscale = wscale;
        a.bias = bias;
        a.out = out;
        a.ldo = ldo;
        a.M = seq;
        a.N = N;
        a.K = K;
        a.act = act;
        a.accumulate = accumulate;
        launch_gemm_i8(a, st);
    });
}

VLA_API int32_t vla_dense_linear_i8_pre_dev(float* out, int32_t ldo, const int8_t* xq, int32_t ldx,
                                            const float* ascale, const int8_t* Wq, int32_t ldw,
                                            const float* wscale, const float* bias, int32_t seq,
                                            int32_t N, int32_t K, int32_t act, int32_t accumulate,
                                            void* stream) {
    return guarded("vla_dense_linear_i8_pre_dev", [&] {
        GemmArgs a{};
        a.A = xq;
        a.lda = ldx;
        a.B = Wq;
        a.ldb = ldw;
        a.ascale = ascale;
        a.wscale = wscale;
        a.bias = bias;
        a.out = out;
        a.ldo = ldo;
        a.M = seq;
        a.N = N;
        a.K = K;
        a.act = act;
        a.accumulate = accumulate;
        launch_gemm_i8(a, as_stream(stream));
    });
}

VLA_API int64_t vla_gemm_i8_split_bytes(int32_t seq, int32_t N, int32_t K) {
    if (seq < 0 || N <= 0 || K <= 0) return -1;
    return (int64_t)gemm_split_bytes(seq, N, K);
}

VLA_API int32_t vla_dense_linear_i8_pre_split_dev(float* out, int32_t ldo, const int8_t* xq, int32_t ldx,
                                                  const float* ascale, const int8_t* Wq, int32_t ldw,
                                                  const float* wscale, const float* bias, int32_t seq,
                                                  int32_t N, int32_t K, int32_t act, int32_t accumulate,
                                                  void* work, int64_t work_bytes, void* stream) {
    return guarded("vla_dense_linear_i8_pre_split_dev", [&] {
        VLA_REQUIRE(work_bytes >= 0 && (work || work_bytes == 0), "bad workspace");
        GemmArgs a{};
        a.A = xq;
        a.lda = ldx;
        a.B = Wq;
        a.ldb = ldw;
        a.ascale = ascale;
        a.wscale = wscale;
        a.bias = bias;
        a.out = out;
        a.ldo = ldo;
        a.M = seq;
        a.N = N;
        a.K = K;
        a.act = act;
        a.accumulate = accumulate;
        a.split_ws = static_cast<int32_t*>(work);
        a.split_bytes = (size_t)work_bytes;
        launch_gemm_i8(a, as_stream(stream));
    });
}

VLA_API int64_t vla_i8_panel_bytes(int32_t seq, int32_t K) {
    if (seq < 0 || seq > kPanelMaxRows || K <= 0) return -1;
    return (int64_t)panel_bytes(seq, K);
}

VLA_API int32_t vla_quantize_act_i8_panel_dev(const float* x, int32_t ldx, int8_t* xq, float* ascale,
                                              int32_t seq, int32_t K, void* stream) {
    return guarded("vla_quantize_act_i8_panel_dev", [&] {
        launch_quantize_rows_panel(x, ldx, xq, ascale, seq, K, as_stream(stream));
    });
}

VLA_API int32_t vla_dense_linear_i8_panel_dev(float* out, int32_t ldo, const int8_t* xq,
                                              const float* ascale, const int8_t* Wq, int32_t ldw,
                                              const float* wscale, const float* bias, int32_t seq,
                                              int32_t N, int32_t K, int32_t act, int32_t accumulate,
                                              void* stream) {
    return guarded("vla_dense_linear_i8_panel_dev", [&] {
        GemmArgs a{};
        a.A = xq;
        a.a_panel = 1;
        a.B = Wq;
        a.ldb = ldw;
        a.ascale = ascale;
        a.wscale = wscale;
        a.bias = bias;
        a.out = out;
        a.ldo = ldo;
        a.M = seq;
        a.N = N;
        a.K = K;
        a.act = act;
        a.accumulate = accumulate;
        launch_gemm_i8(a, as_stream(stream));
    });
}

VLA_API int32_t vla_dense_linear_i8_panel_split_dev(float* out, int32_t ldo, const int8_t* xq,
                                                    const float* ascale, const int8_t* Wq, int32_t ldw,
                                                    const float* wscale, const float* bias, int32_t seq,
                                                    int32_t N, int32_t K, int32_t act, int32_t accumulate,
                                                    void* work, int64_t work_bytes, void* stream) {
    return guarded("vla_dense_linear_i8_panel_split_dev", [&] {
        VLA_REQUIRE(work_bytes >= 0 && (work || work_bytes == 0), "bad workspace");
        GemmArgs a{};
        a.A = xq;
        a.a_panel = 1;
        a.B = Wq;
        a.ldb = ldw;
        a.ascale = ascale;
        a.wscale = wscale;
        a.bias = bias;
        a.out = out;
        a.ldo = ldo;
        a.M = seq;
        a.N = N;
        a.K = K;
        a.act = act;
        a.accumulate = accumulate;
        a.split_ws = static_cast<int32_t*>(work);
        a.split_bytes = (size_t)work_bytes;
        launch_gemm_i8(a, as_stream(stream));
    });
}

static RowQArgs rowop_args(int32_t op, const float* x, int32_t ldx, const float* u, int32_t ldu,
                           const float* w, float eps, int32_t seq, int32_t K) {
    VLA_REQUIRE(op == 0 || op == 2 || op == 3, "row op must be 0 (identity), 2 (RMSNorm) or 3 (silu_gate)");
    RowQArgs r;
    r.op = op;
    r.x = x;
    r.ldx = ldx;
    r.u = op == 3 ? u : nullptr;
    r.ldu = ldu;
    r.w = op == 2 ? w : nullptr;
    r.eps = eps;
    r.rows = seq;
    r.H = K;
    return r;
}

VLA_API int32_t vla_rowop_quantize_i8_panel_dev(int32_t op, const float* x, int32_t ldx, const float* u,
                                                int32_t ldu, const float* w, float eps, int8_t* xq,
                                                float* ascale, int32_t seq, int32_t K, void* stream) {
    return guarded("vla_rowop_quantize_i8_panel_dev", [&] {
        RowQArgs r = rowop_args(op, x, ldx, u, ldu, w, eps, seq, K);
        VLA_REQUIRE(xq && ascale && seq >= 0 && seq <= kPanelMaxRows, "need xq, ascale and seq in [0, 128]");
        r.q = xq;
        r.qs = ascale;
        r.q_panel = 1;
        launch_rowq(r, as_stream(stream));
    });
}

VLA_API int32_t vla_rowop_linear_i8_fits(int32_t op, int32_t seq, int32_t K) {
    return rowop_gemm_fits(op, seq, K) ? 1 : 0;
}

VLA_API int32_t vla_rowop_linear_i8_dev(float* out, int32_t ldo, int32_t op, const float* x, int32_t ldx,
                                        const float* u, int32_t ldu, const float* w, float eps,
                                        const int8_t* Wq, int32_t ldw, const float* wscale, const float* bias,
                                        int32_t seq, int32_t N, int32_t K, int32_t act, int32_t accumulate,
                                        void* stream) {
    return guarded("vla_rowop_linear_i8_dev", [&] {
        const RowQArgs r = rowop_args(op, x, ldx, u, ldu, w, eps, seq, K);
        GemmArgs a{};
        a.B = Wq;
        a.ldb = ldw;
        a.wscale = wscale;
        a.bias = bias;
        a.out = out;
        a.ldo = ldo;
        a.M = seq;
        a.N = N;
        a.K = K;
        a.act = act;
        a.accumulate = accumulate;
        launch_gemm_i8_rowop(r, a, as_stream(stream));
    });
}

VLA_API int32_t vla_gemm_i8_i32_dev(int32_t* acc, const int8_t* xq, int32_t ldx, const int8_t* Wq,
                                    int32_t ldw, int32_t seq, int32_t N, int32_t K, void* stream) {
    return guarded("vla_gemm_i8_i32_dev", [&] {
        VLA_REQUIRE(acc, "null output");
        GemmArgs a{};
        a.A = xq;
        a.lda = ldx;
        a.B = Wq;
        a.ldb = ldw;
        a.acc32 = acc;
        a.M = seq;
        a.N = N;
        a.K = K;
        launch_gemm_i8(a, as_stream(stream));
    });
}

// --------------------------------------------------------- int8 linear --

VLA_API vla_linear_i8* vla_linear_i8_create(const float* W, const float* bias, int32_t N,
                                            int32_t K) {
    vla_linear_i8* out = nullptr;
    guarded("vla_linear_i8_create", [&] { out = Linear::from_f32(W, bias, N, K).release(); });
    return out;
}

VLA_API vla_linear_i8* vla_linear_i8_create_q(const int8_t* Wq, const float* wscale,
                                              const float* bias, int32_t N, int32_t K) {
    vla_linear_i8* out = nullptr;
    guarded("vla_linear_i8_create_q", [&] { out = Linear::from_i8(Wq, K, wscale, bias, N, K).release(); });
    return out;
}

VLA_API void vla_linear_i8_free(vla_linear_i8* lin) { delete lin; }

VLA_API int32_t vla_linear_i8_download(const vla_linear_i8* lin, int8_t* Wq, int32_t ldq, float* wscale) {
    return guarded("vla_linear_i8_download", [&] {
        VLA_REQUIRE(lin, "null linear");
        lin->download(Wq, ldq, wscale);
    });
}

VLA_API int32_t vla_linear_i8_set_bias(vla_linear_i8* lin, const float* bias) {
    return guarded("vla_linear_i8_set_bias", [&] {
        VLA_REQUIRE(lin, "null linear");
        lin->set_bias(bias);
    });
}

// Host-pointer forward over resident weights: only the activations and
// outputs cross PCIe.
static void linear_host(const vla_linear_i8* lin, float* out, const float* x, const int8_t* xq_in, int32_t ldq,
                        int8_t* xq_out, const float* ascale_in, float* ascale_out, int32_t seq) {
    VLA_REQUIRE(lin, "null linear");
    VLA_REQUIRE(seq >= 0, "need seq >= 0");
    const int N = lin->N(), K = lin->K(), Kp = kpad4(K), ldw = lin->ldw();
    VLA_REQUIRE(seq == 0 || (out && (x || (xq_in && ascale_in))), "null buffer");
    VLA_REQUIRE(!(xq_in || xq_out) || ldq >= Kp, "int8 row stride below i8_kpad(K)");
    if (seq == 0) return;
    Staging& S = staging();
    auto lk = S.lock();
    hipStream_t st = library_stream();
    S.reset(align256((size_t)seq * K * 4) + align256((size_t)seq * ldw) + align256((size_t)seq * 4) +
            align256((size_t)seq * N * 4));
    int8_t* dq = S.alloc<int8_t>((size_t)seq * ldw);
    float* ds = S.alloc<float>((size_t)seq);
    float* dout = S.alloc<float>((size_t)seq * N);
    if (x) {
        const float* dx = S.upload(x, (size_t)seq * K, st);
        lin->forward(dout, N, dx, seq, dq, ds, 0, 0, st);
        if (xq_out) VLA_HIP_CHECK(hipMemcpy2DAsync(xq_out, ldq, dq, ldw, Kp, seq, hipMemcpyDeviceToHost, st));
        if (ascale_out) VLA_HIP_CHECK(hipMemcpyAsync(ascale_out, ds, (size_t)seq * 4, hipMemcpyDeviceToHost, st));
    } else {
        // rows of i8_kpad(K) bytes into the resident stride, zero past it
        VLA_HIP_CHECK(hipMemsetAsync(dq, 0, (size_t)seq * ldw, st));
        VLA_HIP_CHECK(hipMemcpy2DAsync(dq, ldw, xq_in, ldq, Kp, seq, hipMemcpyHostToDevice, st));
        count_h2d((size_t)seq * Kp, false);
        VLA_HIP_CHECK(hipMemcpyAsync(ds, ascale_in, (size_t)seq * 4, hipMemcpyHostToDevice, st));
        count_h2d((size_t)seq * 4, false);
        lin->forward_quantized(dout, N, dq, ldw, ds, seq, 0, 0, st);
    }
    VLA_HIP_CHECK(hipMemcpyAsync(out, dout, (size_t)seq * N * 4, hipMemcpyDeviceToHost, st));
    VLA_HIP_CHECK(hipStreamSynchronize(st));
}

VLA_API int32_t vla_linear_i8_forward(const vla_linear_i8* lin, float* out, const float* x, int32_t seq,
                                      int8_t* xq_scratch, int32_t ldq, float* ascale_scratch) {
    return guarded("vla_linear_i8_forward", [&] {
        VLA_REQUIRE(seq == 0 || x, "null activations");
        linear_host(lin, out, x, nullptr, ldq, xq_scratch, nullptr, ascale_scratch, seq);
    });
}

VLA_API int32_t vla_linear_i8_forward_quantized(const vla_linear_i8* lin, float* out, const int8_t* xq, int32_t ldq,
                                                const float* ascale, int32_t seq) {
    return guarded("vla_linear_i8_forward_quantized", [&] {
        VLA_REQUIRE(seq == 0 || (xq && ascale), "null activations");
        linear_host(lin, out, nullptr, xq, ldq, nullptr, ascale, nullptr, seq);
    });
}

VLA_API int64_t vla_h2d_bytes(int32_t weights_only) { return (int64_t)h2d_bytes(weights_only != 0); }
VLA_API const int8_t* vla_linear_i8_weights(const vla_linear_i8* lin) { return lin ? lin->Wq() : nullptr; }
VLA_API const float* vla_linear_i8_wscale(const vla_linear_i8* lin) { return lin ? lin->wscale() : nullptr; }
VLA_API int32_t vla_linear_i8_ldw(const vla_linear_i8* lin) { return lin ? lin->ldw() : 0; }

VLA_API int32_t vla_linear_i8_forward_dev(const vla_linear_i8* lin, float* out, const float* x,
                                          int32_t seq, int8_t* xq_scratch, float* ascale_scratch,
                                          int32_t act, int32_t accumulate, void* stream) {
    return guarded("vla_linear_i8_forward_dev", [&] {
        VLA_REQUIRE(lin, "null linear");
        lin->forward(out, lin->N(), x, seq, xq_scratch, ascale_scratch, act, accumulate, as_stream(stream));
    });
}

VLA_API int32_t vla_linear_i8_forward_quantized_dev(const vla_linear_i8* lin, float* out,
                                                    const int8_t* xq, int32_t ldx,
                                                    const float* ascale, int32_t seq, int32_t act,
                                                    int32_t accumulate, void* stream) {
    return guarded("vla_linear_i8_forward_quantized_dev", [&] {
        VLA_REQUIRE(lin, "null linear");
        lin->forward_quantized(out, lin->N(), xq, ldx, ascale, seq, act, accumulate, as_stream(stream));
    });
}

// ---------------------------------------------------------- convolution --

VLA_API int64_t vla_conv2d_i8_workspace_bytes(int32_t H, int32_t Wd, int32_t Cin, int32_t Cout, int32_t k,
                                              int32_t stride, int32_t pad) {
    int64_t n = -1;
    (void)guarded("vla_conv2d_i8_workspace_bytes", [&] {
        VLA_REQUIRE(Cout > 0, "need Cout > 0");
        n = (int64_t)conv_shape(H, Wd, Cin, k, stride, pad, Cout).work;
    });
    return n;
}

VLA_API int32_t vla_conv2d_i8_dev(const vla_linear_i8* lin, float* out, const float* x, int32_t H, int32_t Wd,
                                  int32_t Cin, int32_t k, int32_t stride, int32_t pad, void* work,
                                  int64_t work_bytes, void* stream) {
    return guarded("vla_conv2d_i8_dev", [&] {
        VLA_REQUIRE(lin, "null weights");
        VLA_REQUIRE((int64_t)k * k * Cin == lin->K(), "the weights' K is not k*k*Cin");
        VLA_REQUIRE(work_bytes >= 0, "negative workspace size");
        ConvArgs a{};
        a.out = out;
        a.x = x;
        a.Wq = lin->Wq();
        a.ldw = lin->ldw();
        a.wscale = lin->wscale();
        a.bias = lin->bias();
        a.H = H;
        a.Wd = Wd;
        a.Cin = Cin;
        a.Cout = lin->N();
        a.k = k;
        a.stride = stride;
        a.pad = pad;
        a.work = work;
        a.work_bytes = (size_t)work_bytes;
        launch_conv2d_i8(a, as_stream(stream));
    });
}

// conv2d_i8 with host activations: weights from a resident layer (lin) or
// uploaded from host rows (Wq [Cout][i8_kpad(K)], wscale, bias)
static void conv_host(const vla_linear_i8* lin, float* out, const float* x, const int8_t* Wq, const float* wscale,
                      const float* bias, int H, int Wd, int Cin, int Cout, int k, int stride, int pad) {
    VLA_REQUIRE(Cout > 0, "need Cout > 0");
    const ConvShape c = conv_shape(H, Wd, Cin, k, stride, pad, Cout);
    VLA_REQUIRE(out && x && (lin || (Wq && wscale)), "null buffer");
    VLA_REQUIRE(!lin || (lin->K() == c.K && lin->N() == Cout), "the weights' shape is not [Cout, k*k*Cin]");
    const int Kp = kpad4(c.K), ldw = (Kp + 63) & ~63;
    const size_t nin = (size_t)H * Wd * Cin, nout = (size_t)c.npix * Cout;
    Staging& S = staging();
    auto lk = S.lock();
    hipStream_t st = library_stream();
    S.reset(align256(nin * 4) + (lin ? 0 : align256((size_t)Cout * ldw) + 2 * align256((size_t)Cout * 4)) +
            align256(nout * 4) + align256(c.work));
    ConvArgs a{};
    a.x = S.upload(x, nin, st);
    if (lin) {
        a.Wq = lin->Wq();
        a.ldw = lin->ldw();
        a.wscale = lin->wscale();
        a.bias = lin->bias();
    } else {
        // [Cout][i8_kpad(K)] rows (vla_pack_weights_i8) into 64-byte rows for the aligned GEMM
        int8_t* w = S.alloc<int8_t>((size_t)Cout * ldw);
        VLA_HIP_CHECK(hipMemsetAsync(w, 0, (size_t)Cout * ldw, st));
        VLA_HIP_CHECK(hipMemcpy2DAsync(w, ldw, Wq, Kp, Kp, Cout, hipMemcpyHostToDevice, st));
        count_h2d((size_t)Cout * Kp, true);
        a.Wq = w;
        a.ldw = ldw;
        a.wscale = S.upload(wscale, (size_t)Cout, st, true);
        a.bias = S.upload(bias, (size_t)Cout, st, true);
    }
    a.out = S.alloc<float>(nout);
    a.H = H;
    a.Wd = Wd;
    a.Cin = Cin;
    a.Cout = Cout;
    a.k = k;
    a.stride = stride;
    a.pad = pad;
    a.work = S.alloc<char>(c.work);
    a.work_bytes = c.work;
    launch_conv2d_i8(a, st);
    VLA_HIP_CHECK(hipMemcpyAsync(out, a.out, nout * 4, hipMemcpyDeviceToHost, st));
    VLA_HIP_CHECK(hipStreamSynchronize(st));
}

VLA_API int32_t vla_conv2d_i8(float* out, const float* x, const int8_t* Wq, const float* wscale,
                              const float* bias, int32_t H, int32_t Wd, int32_t Cin, int32_t Cout, int32_t k,
                              int32_t stride, int32_t pad) {
    return guarded("vla_conv2d_i8", [&] {
        conv_host(nullptr, out, x, Wq, wscale, bias, H, Wd, Cin, Cout, k, stride, pad);
    });
}

VLA_API int32_t vla_conv2d_i8_resident(const vla_linear_i8* lin, float* out, const float* x, int32_t H,
                                       int32_t Wd, int32_t Cin, int32_t k, int32_t stride, int32_t pad) {
    return guarded("vla_conv2d_i8_resident", [&] {
        VLA_REQUIRE(lin, "null weights");
        conv_host(lin, out, x, nullptr, nullptr, nullptr, H, Wd, Cin, lin->N(), k, stride, pad);
    });
}

// ------------------------------------------------------------ attention --

VLA_API int32_t vla_attention_dev(float* out, int32_t ldo, const float* Q, int32_t ldq,
                                  const float* K, int32_t ldk, const float* V, int32_t ldv,
                                  int32_t seq_q, int32_t seq_k, int32_t n_q, int32_t n_kv,
                                  int32_t head_dim, float scale, const vla_mask* mask,
                                  void* stream) {
    return guarded("vla_attention_dev", [&] {
        launch_attention(make_attn(out, ldo, Q, ldq, K, ldk, V, ldv, seq_q, seq_k, n_q, n_kv,
                                   head_dim, scale, mask),
                         as_stream(stream));
    });
}

VLA_API int32_t vla_attention(float* out, const float* Q, const float* K, const float* V,
                              int32_t seq_q, int32_t seq_k, int32_t n_q, int32_t n_kv,
                              int32_t head_dim, float scale, const vla_mask* mask) {
    return guarded("vla_attention", [&] {
        VLA_REQUIRE(seq_q >= 0 && seq_k > 0 && n_q > 0 && n_kv > 0 && head_dim > 0, "bad shape");
        VLA_REQUIRE(out && Q && K && V, "null buffer");
        const int kind = mask ? mask->kind : VLA_MASK_NONE;
        VLA_REQUIRE(kind != VLA_MASK_DENSE || mask->dense, "dense mask missing");
        VLA_REQUIRE(kind != VLA_MASK_GROUPS || (mask->q_group && mask->k_group && mask->allow &&
                                                mask->n_groups > 0 && mask->n_groups <= 256),
                    "group mask incomplete");
        if (kind == VLA_MASK_GROUPS) {
            for (int i = 0; i < seq_q; i++)
                VLA_REQUIRE(mask->q_group[i] < mask->n_groups, "q_group id >= n_groups");
            for (int j = 0; j < seq_k; j++)
                VLA_REQUIRE(mask->k_group[j] < mask->n_groups, "k_group id >= n_groups");
        }
        if (seq_q == 0) return;
        const size_t nqo = (size_t)seq_q * n_q * head_dim, nkv = (size_t)seq_k * n_kv * head_dim;
        Staging& S = staging();
        auto lk = S.lock();
        hipStream_t st = library_stream();
        size_t need = 2 * align256(nqo * 4) + 2 * align256(nkv * 4);
        if (kind == VLA_MASK_DENSE) need += align256((size_t)seq_q * seq_k * 4);
        if (kind == VLA_MASK_GROUPS)
            need += align256(seq_q) + align256(seq_k) + align256((size_t)mask->n_groups * mask->n_groups);
        S.reset(need);
        vla_mask dm{};
        if (mask) dm = *mask;
        const float* dQ = S.upload(Q, nqo, st);
        const float* dK = S.upload(K, nkv, st);
        const float* dV = S.upload(V, nkv, st);
        float* dO = S.alloc<float>(nqo);
        if (kind == VLA_MASK_DENSE) dm.dense = S.upload(mask->dense, (size_t)seq_q * seq_k, st);
        if (kind == VLA_MASK_GROUPS) {
            dm.q_group = S.upload(mask->q_group, (size_t)seq_q, st);
            dm.k_group = S.upload(mask->k_group, (size_t)seq_k, st);
            dm.allow = S.upload(mask->allow, (size_t)mask->n_groups * mask->n_groups, st);
        }
        launch_attention(make_attn(dO, 0, dQ, 0, dK, 0, dV, 0, seq_q, seq_k, n_q, n_kv, head_dim,
                                   scale, mask ? &dm : nullptr),
                         st);
        VLA_HIP_CHECK(hipMemcpyAsync(out, dO, nqo * 4, hipMemcpyDeviceToHost, st));
        VLA_HIP_CHECK(hipStreamSynchronize(st));
    });
}

VLA_API int32_t vla_gqa_attention_masked(float* out, const float* Q, const float* K,
                                         const float* V, int32_t seq_q, int32_t seq_k,
                                         int32_t n_q, int32_t n_kv, int32_t head_dim, float scale,
                                         const float* mask) {
    vla_mask m{};
    m.kind = mask ? VLA_MASK_DENSE : VLA_MASK_NONE;
    m.dense = mask;
    return vla_attention(out, Q, K, V, seq_q, seq_k, n_q, n_kv, head_dim, scale, &m);
}

VLA_API int32_t vla_gqa_attention_dense(float* out, const float* Q, const float* K, const float* V,
                                        int32_t seq_q, int32_t seq_k, int32_t n_q, int32_t n_kv,
                                        int32_t head_dim, float scale) {
    return vla_attention(out, Q, K, V, seq_q, seq_k, n_q, n_kv, head_dim, scale, nullptr);
}

// ---------------------------------------------------------------- norms --

VLA_API int32_t vla_layernorm_dev(float* out, const float* x, const float* w, const float* b,
                                  int32_t seq, int32_t hidden, float eps, void* stream) {
    return guarded("vla_layernorm_dev", [&] { launch_layernorm(out, x, w, b, seq, hidden, eps, as_stream(stream)); });
}

VLA_API int32_t vla_rmsnorm_dev(float* out, const float* x, const float* w, int32_t seq,
                                int32_t hidden, float eps, void* stream) {
    return guarded("vla_rmsnorm_dev", [&] { launch_rmsnorm(out, x, w, seq, hidden, eps, as_stream(stream)); });
}

VLA_API int32_t vla_layernorm(float* out, const float* x, const float* w, const float* b,
                              int32_t seq, int32_t hidden, float eps) {
    return guarded("vla_layernorm", [&] {
        VLA_REQUIRE(seq >= 0 && hidden > 0, "need seq >= 0 and hidden > 0");
        VLA_REQUIRE(seq == 0 || (out && x && w), "null buffer");
        if (seq == 0) return;
        const size_t n = (size_t)seq * hidden;
        Staging& S = staging();
        auto lk = S.lock();
        hipStream_t st = library_stream();
        S.reset(align256(n * 4) + 2 * align256((size_t)hidden * 4));
        float* dx = S.upload(x, n, st);
        const float* dw = S.upload(w, (size_t)hidden, st);
        const float* db = S.upload(b, (size_t)hidden, st);
        launch_layernorm(dx, dx, dw, db, seq, hidden, eps, st);
        VLA_HIP_CHECK(hipMemcpyAsync(out, dx, n * 4, hipMemcpyDeviceToHost, st));
        VLA_HIP_CHECK(hipStreamSynchronize(st));
    });
}

VLA_API int32_t vla_rmsnorm(float* out, const float* x, const float* w, int32_t seq,
                            int32_t hidden, float eps) {
    return guarded("vla_rmsnorm", [&] {
        VLA_REQUIRE(seq >= 0 && hidden > 0, "need seq >= 0 and hidden > 0");
        VLA_REQUIRE(seq == 0 || (out && x && w), "null buffer");
        if (seq == 0) return;
        const size_t n = (size_t)seq * hidden;
        Staging& S = staging();
        auto lk = S.lock();
        hipStream_t st = library_stream();
        S.reset(align256(n * 4) + align256((size_t)hidden * 4));
        float* dx = S.upload(x, n, st);
        const float* dw = S.upload(w, (size_t)hidden, st);
        launch_rmsnorm(dx, dx, dw, seq, hidden, eps, st);
        VLA_HIP_CHECK(hipMemcpyAsync(out, dx, n * 4, hipMemcpyDeviceToHost, st));
        VLA_HIP_CHECK(hipStreamSynchronize(st));
    });
}

VLA_API int32_t vla_rope_neox_dev(float* x, int32_t ld, const int32_t* pos, int32_t seq,
                                  int32_t n_heads, int32_t head_dim, float base, void* stream) {
    return guarded("vla_rope_neox_dev", [&] {
        launch_rope_neox(x, ld ? ld : n_heads * head_dim, pos, seq, n_heads, head_dim, base, as_stream(stream));
    });
}

VLA_API int32_t vla_rope_neox(float* x, const int32_t* pos, int32_t seq, int32_t n_heads,
                              int32_t head_dim, float base) {
    return guarded("vla_rope_neox", [&] {
        VLA_REQUIRE(seq >= 0 && n_heads > 0 && head_dim > 0, "bad shape");
        VLA_REQUIRE(seq == 0 || (x && pos), "null buffer");
        if (seq == 0) return;
        const size_t n = (size_t)seq * n_heads * head_dim;
        Staging& S = staging();
        auto lk = S.lock();
        hipStream_t st = library_stream();
        S.reset(align256(n * 4) + align256((size_t)seq * 4));
        float* dx = S.upload(x, n, st);
        const int32_t* dp = S.upload(pos, (size_t)seq, st);
        launch_rope_neox(dx, n_heads * head_dim, dp, seq, n_heads, head_dim, base, st);
        VLA_HIP_CHECK(hipMemcpyAsync(x, dx, n * 4, hipMemcpyDeviceToHost, st));
        VLA_HIP_CHECK(hipStreamSynchronize(st));
    });
}

// ------------------------------------------------------------- eltwise --

static int32_t act_host(const char* where, float* x, int32_t n, int act) {
    return guarded(where, [&] {
        VLA_REQUIRE(n >= 0, "n < 0");
        VLA_REQUIRE(n == 0 || x, "null buffer");
        if (n == 0) return;
        Staging& S = staging();
        auto lk = S.lock();
        hipStream_t st = library_stream();
        S.reset(align256((size_t)n * 4));
        float* dx = S.upload(x, (size_t)n, st);
        launch_act(dx, n, act, st);
        VLA_HIP_CHECK(hipMemcpyAsync(x, dx, (size_t)n * 4, hipMemcpyDeviceToHost, st));
        VLA_HIP_CHECK(hipStreamSynchronize(st));
    });
}

VLA_API int32_t vla_gelu_tanh(float* x, int32_t n) { return act_host("vla_gelu_tanh", x, n, VLA_ACT_GELU_TANH); }
VLA_API int32_t vla_gelu_erf(float* x, int32_t n) { return act_host("vla_gelu_erf", x, n, VLA_ACT_GELU_ERF); }
VLA_API int32_t vla_relu(float* x, int32_t n) { return act_host("vla_relu", x, n, VLA_ACT_RELU); }

VLA_API int32_t vla_silu_gate(float* out, const float* g, const float* u, int32_t n) {
    return guarded("vla_silu_gate", [&] {
        VLA_REQUIRE(n >= 0, "n < 0");
        VLA_REQUIRE(n == 0 || (out && g && u), "null buffer");
        if (n == 0) return;
        Staging& S = staging();
        auto lk = S.lock();
        hipStream_t st = library_stream();
        S.reset(2 * align256((size_t)n * 4));
        float* dg = S.upload(g, (size_t)n, st);
        const float* du = S.upload(u, (size_t)n, st);
        launch_silu_gate(dg, dg, du, n, st);
        VLA_HIP_CHECK(hipMemcpyAsync(out, dg, (size_t)n * 4, hipMemcpyDeviceToHost, st));
        VLA_HIP_CHECK(hipStreamSynchronize(st));
    });
}

VLA_API int32_t vla_gelu_tanh_dev(float* x, int64_t n, void* stream) {
    return guarded("vla_gelu_tanh_dev", [&] { launch_act(x, n, VLA_ACT_GELU_TANH, as_stream(stream)); });
}
VLA_API int32_t vla_gelu_erf_dev(float* x, int64_t n, void* stream) {
    return guarded("vla_gelu_erf_dev", [&] { launch_act(x, n, VLA_ACT_GELU_ERF, as_stream(stream)); });
}
VLA_API int32_t vla_relu_dev(float* x, int64_t n, void* stream) {
    return guarded("vla_relu_dev", [&] { launch_act(x, n, VLA_ACT_RELU, as_stream(stream)); });
}
VLA_API int32_t vla_silu_gate_dev(float* out, const float* g, const float* u, int64_t n,
                                  void* stream) {
    return guarded("vla_silu_gate_dev", [&] { launch_silu_gate(out, g, u, n, as_stream(stream)); });
}
VLA_API int32_t vla_add_dev(float* out, const float* a, const float* b, int64_t n, void* stream) {
    return guarded("vla_add_dev", [&] { launch_add(out, a, b, n, as_stream(stream)); });
}

// ------------------------------------------------------- fp32 linear --

VLA_API int32_t vla_dense_linear(float* out, const float* x, const float* W, const float* bias,
                                 int32_t seq, int32_t N, int32_t K) {
    return guarded("vla_dense_linear", [&] {
        VLA_REQUIRE(seq >= 0 && N > 0 && K > 0, "need seq >= 0, N > 0 and K > 0");
        VLA_REQUIRE(seq == 0 || (out && x && W), "null buffer");
        if (seq == 0) return;
        Staging& S = staging();
        auto lk = S.lock();
        hipStream_t st = library_stream();
        S.reset(align256((size_t)seq * K * 4) + align256((size_t)N * K * 4) + align256((size_t)N * 4) +
                align256((size_t)seq * N * 4));
        const float* dx = S.upload(x, (size_t)seq * K, st);
        const float* dW = S.upload(W, (size_t)N * K, st, true);
        const float* db = S.upload(bias, (size_t)N, st, true);
        float* dout = S.alloc<float>((size_t)seq * N);
        launch_linear_f32(dout, N, dx, K, dW, K, db, seq, N, K, 0, 0, 1.0f, st);
        VLA_HIP_CHECK(hipMemcpyAsync(out, dout, (size_t)seq * N * 4, hipMemcpyDeviceToHost, st));
        VLA_HIP_CHECK(hipStreamSynchronize(st));
    });
}

VLA_API int32_t vla_dense_linear_dev(float* out, int32_t ldo, const float* x, int32_t ldx,
                                     const float* W, int32_t ldw, const float* bias, int32_t seq,
                                     int32_t N, int32_t K, int32_t act, int32_t accumulate,
                                     float alpha, void* stream) {
    return guarded("vla_dense_linear_dev", [&] {
        launch_linear_f32(out, ldo, x, ldx, W, ldw, bias, seq, N, K, act, accumulate, alpha,
                          as_stream(stream));
    });
}

}  // extern "C"
