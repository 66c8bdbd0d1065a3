// linear.h - device-resident int8 linear layer: the MI355X form of the int8
// state nn::Linear keeps after init_int8 (src/nn/linear.h:40-48, 85-99;
// src/nn/linear.cpp:66-133, 170-172).
//
// Weights live in HBM as int8 rows [N][ldw] (ldw = i8_kpad(K) rounded up to
// 64 bytes, zero past K), per-output-channel fp32 scales [N] and an optional
// fp32 bias [N]. They are uploaded (and, from fp32, quantized on the device
// with the pack_weights_i8 formula) once; forward() only streams them.
#pragma once

#include "common.h"

#include <memory>

struct vla_linear_i8 {
    // Linear::init + init_int8 from fp32 W [N,K] (host). K bound as
    // linear.cpp:67; any N (the GPU layout has no 16-row panels).
    static std::unique_ptr<vla_linear_i8> from_f32(const float* W, const float* bias, int N, int K);
    // From int8 rows Wq [N, ldq] (host, ldq >= K, bytes past K ignored) + wscale [N].
    static std::unique_ptr<vla_linear_i8> from_i8(const int8_t* Wq, int ldq, const float* wscale,
                                                  const float* bias, int N, int K);
    ~vla_linear_i8();
    vla_linear_i8(const vla_linear_i8&) = delete;
    vla_linear_i8& operator=(const vla_linear_i8&) = delete;

    int N() const { return N_; }
    int K() const { return K_; }
    int ldw() const { return ldw_; }
    const int8_t* Wq() const { return Wq_; }
    const float* wscale() const { return wscale_; }
    const float* bias() const { return bias_; }

    // The resident rows and scales copied to the host: Wq [N, ldq] (ldq >=
    // i8_kpad(K); bytes [K, ldq) zero), wscale [N].
    void download(int8_t* Wq, int ldq, float* wscale) const;
    // Replace the bias with host [N] values, or drop it (null).
    void set_bias(const float* bias);

    // out [seq, ldo] = x [seq, K] W^T + bias, quantizing x into xq [seq, ldw] /
    // ascale [seq] first (Linear::forward's int8 branch, linear.cpp:121-133).
    void forward(float* out, int ldo, const float* x, int seq, int8_t* xq, float* ascale,
                 int act, int accumulate, hipStream_t st) const;
    // Activations already quantized, xq [seq, ldx] (Linear::forward_quantized).
    void forward_quantized(float* out, int ldo, const int8_t* xq, int ldx, const float* ascale,
                           int seq, int act, int accumulate, hipStream_t st) const;

private:
    vla_linear_i8() = default;
    void alloc(int N, int K, bool has_bias);
    int N_ = 0, K_ = 0, ldw_ = 0;
    int8_t* Wq_ = nullptr;
    float* wscale_ = nullptr;
    float* bias_ = nullptr;
};

namespace vla {
namespace hip {
using Linear = ::vla_linear_i8;
}  // namespace hip
}  // namespace vla
