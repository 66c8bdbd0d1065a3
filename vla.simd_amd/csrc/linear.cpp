// linear.cpp - device-resident int8 linear (see linear.h).
#include "linear.h"

#include "runtime.h"

#include <cstring>

using namespace vla::hip;

void vla_linear_i8::alloc(int N, int K, bool has_bias) {
    VLA_REQUIRE(N > 0 && K > 0, "linear: need N > 0 and K > 0");
    VLA_REQUIRE(K <= kMaxI8K, "linear: K exceeds the int8 accumulator bound INT_MAX/(255*127)");
    N_ = N;
    K_ = K;
    ldw_ = round_up(kpad4(K), 64);
    VLA_HIP_CHECK(hipMalloc(&Wq_, (size_t)N * ldw_));
    VLA_HIP_CHECK(hipMalloc(&wscale_, (size_t)N * 4));
    if (has_bias) VLA_HIP_CHECK(hipMalloc(&bias_, (size_t)N * 4));
}

vla_linear_i8::~vla_linear_i8() {
    // destructors must not throw; a failed free is left to process teardown
    if (Wq_) (void)hipFree(Wq_);
    if (wscale_) (void)hipFree(wscale_);
    if (bias_) (void)hipFree(bias_);
}

std::unique_ptr<vla_linear_i8> vla_linear_i8::from_f32(const float* W, const float* bias, int N,
                                                       int K) {
    VLA_REQUIRE(W, "linear: null weights");
    std::unique_ptr<vla_linear_i8> L(new vla_linear_i8());
    L->alloc(N, K, bias != nullptr);
    float* dW = nullptr;
    VLA_HIP_CHECK(hipMalloc(&dW, (size_t)N * K * 4));
    try {
        VLA_HIP_CHECK(hipMemcpy(dW, W, (size_t)N * K * 4, hipMemcpyHostToDevice));
        count_h2d((size_t)N * K * 4 + (bias ? (size_t)N * 4 : 0), true);
        // pack_weights_i8 (gemm_i8.cpp:56-89) is the activation quantizer's
        // formula applied per output row; it also zero-fills [K, ldw).
        launch_quantize_rows(dW, K, L->Wq_, L->ldw_, L->wscale_, N, K, nullptr);
        if (bias) VLA_HIP_CHECK(hipMemcpy(L->bias_, bias, (size_t)N * 4, hipMemcpyHostToDevice));
        VLA_HIP_CHECK(hipDeviceSynchronize());
    } catch (...) {
        (void)hipFree(dW);
        throw;
    }
    VLA_HIP_CHECK(hipFree(dW));
    return L;
}

std::unique_ptr<vla_linear_i8> vla_linear_i8::from_i8(const int8_t* Wq, int ldq, const float* wscale,
                                                      const float* bias, int N, int K) {
    VLA_REQUIRE(Wq && wscale, "linear: null weights or scales");
    VLA_REQUIRE(ldq >= K, "linear: int8 row stride below K");
    std::unique_ptr<vla_linear_i8> L(new vla_linear_i8());
    L->alloc(N, K, bias != nullptr);
    VLA_HIP_CHECK(hipMemset(L->Wq_, 0, (size_t)N * L->ldw_));
    VLA_HIP_CHECK(hipMemcpy2D(L->Wq_, L->ldw_, Wq, ldq, K, N, hipMemcpyHostToDevice));
    VLA_HIP_CHECK(hipMemcpy(L->wscale_, wscale, (size_t)N * 4, hipMemcpyHostToDevice));
    if (bias) VLA_HIP_CHECK(hipMemcpy(L->bias_, bias, (size_t)N * 4, hipMemcpyHostToDevice));
    count_h2d((size_t)N * K + (size_t)N * 4 * (bias ? 2 : 1), true);
    VLA_HIP_CHECK(hipDeviceSynchronize());
    return L;
}

void vla_linear_i8::download(int8_t* Wq, int ldq, float* wscale) const {
    VLA_REQUIRE(Wq && wscale, "linear: null output");
    VLA_REQUIRE(ldq >= kpad4(K_), "linear: row stride below i8_kpad(K)");
    // resident rows hold zeros in [K, ldw); a wider host stride gets zeros too
    const int w = ldq < ldw_ ? ldq : ldw_;
    VLA_HIP_CHECK(hipMemcpy2D(Wq, ldq, Wq_, ldw_, w, N_, hipMemcpyDeviceToHost));
    if (ldq > w)
        for (int n = 0; n < N_; n++) std::memset(Wq + (size_t)n * ldq + w, 0, (size_t)(ldq - w));
    VLA_HIP_CHECK(hipMemcpy(wscale, wscale_, (size_t)N_ * 4, hipMemcpyDeviceToHost));
}

void vla_linear_i8::set_bias(const float* bias) {
    if (!bias) {
        if (bias_) VLA_HIP_CHECK(hipFree(bias_));
        bias_ = nullptr;
        return;
    }
    if (!bias_) VLA_HIP_CHECK(hipMalloc(&bias_, (size_t)N_ * 4));
    VLA_HIP_CHECK(hipMemcpy(bias_, bias, (size_t)N_ * 4, hipMemcpyHostToDevice));
    count_h2d((size_t)N_ * 4, true);
}

void vla_linear_i8::forward(float* out, int ldo, const float* x, int seq, int8_t* xq, float* ascale,
                            int act, int accumulate, hipStream_t st) const {
    if (seq == 0) return;
    launch_quantize_rows(x, K_, xq, ldw_, ascale, seq, K_, st);
    forward_quantized(out, ldo, xq, ldw_, ascale, seq, act, accumulate, st);
}

void vla_linear_i8::forward_quantized(float* out, int ldo, const int8_t* xq, int ldx,
                                      const float* ascale, int seq, int act, int accumulate,
                                      hipStream_t st) const {
    GemmArgs a{};
    a.A = xq;
    a.lda = ldx;
    a.B = Wq_;
    a.ldb = ldw_;
    a.ascale = ascale;
    a.wscale = wscale_;
    a.bias = bias_;
    a.out = out;
    a.ldo = ldo;
    a.M = seq;
    a.N = N_;
    a.K = K_;
    a.act = act;
    a.accumulate = accumulate;
    launch_gemm_i8(a, st);
}
