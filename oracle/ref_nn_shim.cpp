/*
 * ref_nn_shim.cpp - extern "C" entry points that drive the REFERENCE's own
 * nn::Linear and nn::MhaQKV (src/nn/linear.cpp, src/nn/attention.cpp) on
 * whichever op backend the library is linked with:
 *   _ref/libvla_ref.so      the reference's CPU backend (AVX2 / AVX-VNNI)
 *   _ref/libvla_ref_hip.so  vla.simd_amd/hal/ops_hip.cpp, i.e. libvla_simd_hip.so
 * so one test can run the reference's layer code on both and compare.
 *
 * TEST INFRASTRUCTURE ONLY; the product never loads it.
 */
#include "models/diffusion/unet1d.h"
#include "nn/attention.h"
#include "nn/conv.h"
#include "nn/linear.h"
#include "ops/quant_ops.h"

#include <cstdio>
#include <cstring>
#include <exception>
#include <memory>
#include <vector>

#define REF_API extern "C" __attribute__((visibility("default")))

using namespace tcpu;

/* nn::Linear(W [N, K], b [N], Role::Gemm), init_int8 when int8 != 0, then
 * forward(out [seq, N], x [seq, K]). Returns 1 if the layer is int8, 0 if
 * fp32, -1 on an exception. */
REF_API int ref_nn_linear_forward(const float* W, const float* b, int N, int K, int int8, const float* x,
                                  int seq, float* out) {
    try {
        nn::Linear lin;
        lin.init(W, b, N, K, nn::Linear::Role::Gemm);
        const bool q = int8 && lin.init_int8();
        lin.forward(out, x, seq);
        return q ? 1 : 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_nn_linear_forward: %s\n", e.what());
        return -1;
    }
}

/* test_ops.cpp:195-220's layer: an nn::MhaQKV of `heads` heads over dim whose
 * four projections all take W [dim, dim] and b [dim] (int8 when int8 != 0),
 * run as forward(out, xq, xk, xv, rows, seq_kv): inputs that alias take the
 * shared-quantization branches (attention.cpp:40-59). q/k/v get the projected
 * rows the attention read (Scratch q, k, v). Returns 0, or -1 on an exception. */
REF_API int ref_nn_mha_forward(int dim, int heads, const float* W, const float* b, int int8, const float* xq,
                               const float* xk, const float* xv, int rows, int seq_kv, float* out, float* q,
                               float* k, float* v) {
    try {
        nn::MhaQKV layer;
        layer.set_shape(heads, dim / heads);
        for (nn::Linear* lin : {&layer.wq, &layer.wk, &layer.wv, &layer.wo}) {
            lin->init(W, b, dim, dim, nn::Linear::Role::Gemm);
            if (int8) lin->init_int8();
        }
        nn::Scratch s;
        layer.forward(out, xq, xk, xv, rows, seq_kv, s);
        std::memcpy(q, s.q.data(), (size_t)rows * dim * sizeof(float));
        std::memcpy(v, s.v.data(), (size_t)seq_kv * dim * sizeof(float));
        if (!layer.wk.kt_ok()) std::memcpy(k, s.k.data(), (size_t)seq_kv * dim * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_nn_mha_forward: %s\n", e.what());
        return -1;
    }
}

/* Layers that live across calls (a model's layers are loaded once and run
 * many times): nn::Linear, nn::MhaQKV and nn::Conv2d with their weights
 * (the layers keep raw pointers to W and b, so the handle owns copies). */
struct NnLinear {
    std::vector<float> W, b;
    nn::Linear lin;
    bool q = false;
};

REF_API void* ref_nn_linear_load(const float* W, const float* b, int N, int K, int int8, int* is_int8) {
    try {
        auto h = std::make_unique<NnLinear>();
        h->W.assign(W, W + (size_t)N * K);
        if (b) h->b.assign(b, b + N);
        h->lin.init(h->W.data(), b ? h->b.data() : nullptr, N, K, nn::Linear::Role::Gemm);
        h->q = int8 && h->lin.init_int8();
        *is_int8 = h->q ? 1 : 0;
        return h.release();
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_nn_linear_load: %s\n", e.what());
        return nullptr;
    }
}

/* forward (linear.cpp:121-133), or with quantized input (xq [seq,
 * i8_kpad(K)], scales [seq]) forward_quantized (:170-172) */
REF_API int ref_nn_linear_run(void* h, const float* x, const int8_t* xq, const float* scales, int seq, float* out) {
    try {
        auto* l = static_cast<NnLinear*>(h);
        if (xq) l->lin.forward_quantized(out, xq, scales, seq);
        else l->lin.forward(out, x, seq);
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_nn_linear_run: %s\n", e.what());
        return -1;
    }
}

REF_API void ref_nn_linear_free(void* h) { delete static_cast<NnLinear*>(h); }

struct NnMha {
    std::vector<float> W, b;
    nn::MhaQKV layer;
    nn::Scratch s;
};

REF_API void* ref_nn_mha_load(int dim, int heads, const float* W, const float* b, int int8) {
    try {
        auto h = std::make_unique<NnMha>();
        h->W.assign(W, W + (size_t)dim * dim);
        h->b.assign(b, b + dim);
        h->layer.set_shape(heads, dim / heads);
        for (nn::Linear* lin : {&h->layer.wq, &h->layer.wk, &h->layer.wv, &h->layer.wo}) {
            lin->init(h->W.data(), h->b.data(), dim, dim, nn::Linear::Role::Gemm);
            if (int8) lin->init_int8();
        }
        return h.release();
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_nn_mha_load: %s\n", e.what());
        return nullptr;
    }
}

REF_API int ref_nn_mha_run(void* h, const float* xq, const float* xk, const float* xv, int rows, int seq_kv,
                           float* out) {
    try {
        auto* m = static_cast<NnMha*>(h);
        m->layer.forward(out, xq, xk, xv, rows, seq_kv, m->s);
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_nn_mha_run: %s\n", e.what());
        return -1;
    }
}

REF_API void ref_nn_mha_free(void* h) { delete static_cast<NnMha*>(h); }

struct NnConv {
    std::vector<float> W, b;
    nn::Conv2d conv;
    bool q = false;
};

/* nn::Conv2d (conv.cpp): W [Cout, k, k, Cin], init_int8 when int8 != 0 */
REF_API void* ref_nn_conv_load(const float* W, const float* b, int Cout, int k, int Cin, int int8, int* is_int8) {
    try {
        auto h = std::make_unique<NnConv>();
        h->W.assign(W, W + (size_t)Cout * k * k * Cin);
        if (b) h->b.assign(b, b + Cout);
        h->conv.init(h->W.data(), b ? h->b.data() : nullptr, Cout, k, Cin);
        h->q = int8 && h->conv.init_int8();
        *is_int8 = h->q ? 1 : 0;
        return h.release();
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_nn_conv_load: %s\n", e.what());
        return nullptr;
    }
}

REF_API int ref_nn_conv_run(void* h, const float* x, int H, int Wd, int stride, int pad, float* out) {
    try {
        static_cast<NnConv*>(h)->conv.forward(out, x, H, Wd, stride, pad);
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_nn_conv_run: %s\n", e.what());
        return -1;
    }
}

REF_API void ref_nn_conv_free(void* h) { delete static_cast<NnConv*>(h); }

/* The backend's pack + pre kernel against its scalar statement of the same
 * call (test_ops.cpp:138-157): W [N, K] fp32 packed by pack_weights_i8, x
 * quantized by quantize_act_i8; pre [seq, N] from dense_linear_i8_pre, ref
 * from dense_linear_i8_ref. Returns 0, or -1 on an exception. */
REF_API int ref_nn_pre_vs_ref(const float* W, int N, int K, const float* x, int seq, const float* bias, float* pre,
                              float* ref) {
    try {
        std::vector<int32_t> packed(packed_i8_words(N, K));
        std::vector<float> ws(N), as(seq);
        std::vector<int8_t> xq((size_t)seq * i8_kpad(K));
        pack_weights_i8(W, (int8_t*)packed.data(), ws.data(), N, K);
        quantize_act_i8(x, xq.data(), as.data(), seq, K);
        dense_linear_i8_pre(pre, xq.data(), as.data(), (const int8_t*)packed.data(), ws.data(), bias, seq, N, K);
        dense_linear_i8_ref(ref, xq.data(), as.data(), (const int8_t*)packed.data(), ws.data(), bias, seq, N, K);
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_nn_pre_vs_ref: %s\n", e.what());
        return -1;
    }
}

/* Diffusion Policy's noise-prediction UNet (src/models/diffusion/unet1d.cpp)
 * loaded from <dir>/unet.bin with its W8A8 GEMMs when int8 != 0
 * (diffusion_model.cpp:113-114: the Gemm-role conv / residual / downsample
 * linears). cfg[12] = {action_dim, horizon, down0, down1, down2, kernel_size,
 * n_groups, step_embed_dim, film_scale, state_dim, n_cams, num_keypoints};
 * n_obs_steps 2. Returns the handle (null on failure); n_int8 gets the count. */
REF_API void* ref_unet_load(const char* dir, const int* cfg, int int8, int* n_int8) {
    try {
        DPConfig c;
        c.action_dim = cfg[0];
        c.horizon = cfg[1];
        c.down_dims = {cfg[2], cfg[3], cfg[4]};
        c.kernel_size = cfg[5];
        c.n_groups = cfg[6];
        c.step_embed_dim = cfg[7];
        c.film_scale = cfg[8] != 0;
        c.state_dim = cfg[9];
        c.n_cams = cfg[10];
        c.num_keypoints = cfg[11];
        c.n_obs_steps = 2;
        auto* u = new DPUNet1d();
        if (!u->load(dir, "unet", c, int8 != 0)) {
            delete u;
            return nullptr;
        }
        *n_int8 = u->n_int8;
        return u;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_unet_load: %s\n", e.what());
        return nullptr;
    }
}

REF_API void ref_unet_free(void* h) { delete static_cast<DPUNet1d*>(h); }

/* eps [horizon, action_dim] = UNet(sample [horizon, action_dim], gc [global_cond_dim], t) */
REF_API int ref_unet_forward(void* h, float* eps, const float* sample, const float* gc, int t) {
    try {
        static_cast<DPUNet1d*>(h)->forward(eps, sample, gc, t);
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_unet_forward: %s\n", e.what());
        return -1;
    }
}
