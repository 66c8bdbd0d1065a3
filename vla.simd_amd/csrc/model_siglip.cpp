// model_siglip.cpp - SmolVLA's SigLIP vision tower and connector on the
// device (see models.h).
//
// Follows src/models/smolvla/siglip_vision.cpp: load() :21-140 reads vit.meta
// and vit.bin (an fp32 region, then bf16 weights); encode() :151-202 extracts
// the patches, runs the patch linear, adds the positions, runs n_layers
// nn::EncoderLayer::forward (src/nn/encoder.cpp:26-77, full attention, GELU
// tanh), the post-LayerNorm, the pixel shuffle and the bias-free modality
// projection. Value-preserving regroupings:
//   - the positional rows are copied into x first and the patch linear adds
//     its output into them in its epilogue (proj + pos and pos + proj are the
//     same IEEE sum);
//   - q|k|v read one LayerNorm output, so they are one row-concatenated layer
//     behind one quantization (the same bytes and scales three separate int8
//     layers compute from that input);
//   - the wo and w2 residual adds and the gelu after w1 are GEMM epilogues
//     (x + proj, encoder.cpp:47-48 / 73-74, is the add the epilogue makes).
#include "ckpt.h"
#include "models.h"

#include <cmath>

namespace vla {
namespace hip {

namespace {

int vit_int(const std::map<std::string, double>& m, const char* k, int def) {
    return vla::hip::meta_int(m, "vit.meta", k, def);
}

}  // namespace

SiglipTf::SiglipTf(const std::string& dir, int int8_mask) {
    const CkptFiles files(dir);  // a converted directory or a vla.simd GGUF
    const auto m = files.meta("vit.meta");
    H_ = vit_int(m, "hidden", H_);
    heads_ = vit_int(m, "n_heads", heads_);
    hd_ = vit_int(m, "head_dim", hd_);
    I_ = vit_int(m, "inter", I_);
    NL_ = vit_int(m, "n_layers", NL_);
    P_ = vit_int(m, "patch", P_);
    img_ = vit_int(m, "img", img_);
    NP_ = vit_int(m, "n_patches", NP_);
    sf_ = vit_int(m, "scale_factor", sf_);
    mm_out_ = vit_int(m, "mm_out", mm_out_);
    ntok_ = vit_int(m, "n_img_tok", ntok_);
    if (m.count("ln_eps")) eps_ = (float)m.at("ln_eps");
    // siglip_vision.cpp:43-70: the grids must close
    side_ = (int)std::lround(std::sqrt((double)std::max(NP_, 0)));
    VLA_REQUIRE(H_ > 0 && heads_ > 0 && hd_ > 0 && heads_ * hd_ == H_ && I_ > 0 && NL_ >= 1 && P_ > 0 &&
                    img_ > 0 && NP_ > 0 && sf_ > 0 && mm_out_ > 0 && std::isfinite(eps_) && eps_ > 0 &&
                    side_ * side_ == NP_ && img_ % P_ == 0 && (img_ / P_) * (img_ / P_) == NP_ &&
                    side_ % sf_ == 0 && (side_ / sf_) * (side_ / sf_) == ntok_,
                "vit.meta: shapes do not close (siglip_vision.cpp:43-70 bounds)");
    VLA_REQUIRE(P_ % 4 == 0 && H_ % 4 == 0 && NP_ < 65536 && (int64_t)H_ * sf_ * sf_ < (1 << 30),
                "vit.meta: the device path needs patch and hidden multiples of 4");
    const int H = H_, I = I_, PD = 3 * P_ * P_, SD = H * sf_ * sf_;

    const std::vector<char> raw = files.bytes("vit.bin");
    const size_t fcount = (size_t)H + (size_t)NP_ * H + (size_t)NL_ * (8 * (size_t)H + I + H) + 2 * (size_t)H;
    const size_t wcount = (size_t)H * PD + (size_t)NL_ * (4 * (size_t)H * H + 2 * (size_t)I * H) +
                          (size_t)mm_out_ * SD;
    VLA_REQUIRE(raw.size() == fcount * 4 + wcount * 2, "vit.bin: size does not match vit.meta");
    const float* fp = reinterpret_cast<const float*>(raw.data());
    const uint16_t* wb = reinterpret_cast<const uint16_t*>(raw.data() + fcount * 4);
    auto f32 = [&](size_t n) {
        const float* r = fp;
        fp += n;
        return r;
    };
    std::vector<float> tmp;
    auto bf = [&](size_t n) {  // next n bf16 weights as fp32 (Linear::init_int8 widens them the same way)
        tmp.resize(n);
        for (size_t i = 0; i < n; i++) tmp[i] = bf16_to_f32(wb[i]);
        wb += n;
        return tmp;
    };

    const bool ia = int8_mask & 1, i1 = int8_mask & 2, i2 = int8_mask & 4, ip = int8_mask & 8;
    const float* patch_b = f32(H);
    pos_ = A_.upload(f32((size_t)NP_ * H), (size_t)NP_ * H);
    struct LayerF {
        const float *ln1s, *ln1b, *bq, *bk, *bv, *bo, *ln2s, *ln2b, *b1, *b2;
    };
    std::vector<LayerF> lf(NL_);
    for (LayerF& f : lf) {
        f.ln1s = f32(H);
        f.ln1b = f32(H);
        f.bq = f32(H);
        f.bk = f32(H);
        f.bv = f32(H);
        f.bo = f32(H);
        f.ln2s = f32(H);
        f.ln2b = f32(H);
        f.b1 = f32(I);
        f.b2 = f32(H);
    }
    post_s_ = A_.upload(f32(H), H);
    post_b_ = A_.upload(f32(H), H);

    {
        const std::vector<float> w = bf((size_t)H * PD);
        patch_.init(A_, w.data(), patch_b, H, PD, ip);
    }
    layers_.resize(NL_);
    for (int L = 0; L < NL_; L++) {
        Layer& e = layers_[L];
        const LayerF& f = lf[L];
        e.ln1s = A_.upload(f.ln1s, H);
        e.ln1b = A_.upload(f.ln1b, H);
        e.ln2s = A_.upload(f.ln2s, H);
        e.ln2b = A_.upload(f.ln2b, H);
        const std::vector<float> q = bf((size_t)H * H), k = bf((size_t)H * H), v = bf((size_t)H * H);
        e.qkv.init(A_, {{q.data(), f.bq, H}, {k.data(), f.bk, H}, {v.data(), f.bv, H}}, H, ia);
        const std::vector<float> o = bf((size_t)H * H);
        e.o.init(A_, o.data(), f.bo, H, H, ia);
        const std::vector<float> w1 = bf((size_t)I * H);
        e.w1.init(A_, w1.data(), f.b1, I, H, i1);
        const std::vector<float> w2 = bf((size_t)H * I);
        e.w2.init(A_, w2.data(), f.b2, H, I, i2);
        n_int8_ += (ia ? 4 : 0) + i1 + i2;
    }
    {
        const std::vector<float> w = bf((size_t)mm_out_ * SD);
        mm_.init(A_, w.data(), nullptr, mm_out_, SD, ip);
    }
    n_int8_ += ip ? 2 : 0;

    // activations: every shape is fixed by the checkpoint
    patches_ = A_.alloc<float>((size_t)NP_ * PD);
    x_ = A_.alloc<float>((size_t)NP_ * H);
    h_ = A_.alloc<float>((size_t)NP_ * H);
    qkv_ = A_.alloc<float>((size_t)NP_ * 3 * H);
    att_ = A_.alloc<float>((size_t)NP_ * H);
    ff_ = A_.alloc<float>((size_t)NP_ * I);
    shuf_ = A_.alloc<float>((size_t)ntok_ * SD);
    out_ = A_.alloc<float>((size_t)ntok_ * mm_out_);
    int maxld = 0;
    for (int k : {H, I, PD, SD}) maxld = std::max(maxld, round_up(kpad4(k), 64));
    ctx_.alloc(A_, NP_, maxld);
    VLA_HIP_CHECK(hipStreamCreateWithFlags(&own_, hipStreamNonBlocking));
}

SiglipTf::~SiglipTf() {
    if (own_) (void)hipStreamDestroy(own_);
}

void SiglipTf::run(hipStream_t st) {
    Ctx c = ctx_;
    c.st = st;
    const int H = H_, T = NP_;
    const float scale = 1.0f / std::sqrt((float)hd_);
    const MaskSpec full;  // kind 0: SigLIP attends over every patch (encode :166-167)

    // patch embedding + positions (:156-164)
    copy_f32(x_, pos_, (int64_t)T * H, st);
    linear(c, patch_, x_, H, patches_, 3 * P_ * P_, T, 0, 1);

    auto ln_for = [&](const float* w, const float* b, const DLinear& L) {
        RowQArgs r;
        r.op = 1;
        r.x = x_;
        r.ldx = H;
        r.w = w;
        r.b = b;
        r.eps = eps_;
        r.rows = T;
        r.H = H;
        return rowop_for(c, L, r, L.int8() ? nullptr : h_, H, 0);
    };
    for (const Layer& L : layers_) {
        const In h1 = ln_for(L.ln1s, L.ln1b, L.qkv);
        linear(c, L.qkv, h1, qkv_, 3 * H, T);
        attend(st, att_, H, qkv_, 3 * H, qkv_ + H, 3 * H, qkv_ + 2 * H, 3 * H, T, T, heads_, heads_, hd_, scale,
               full);
        linear(c, L.o, x_, H, att_, H, T, 0, 1);
        const In h2 = ln_for(L.ln2s, L.ln2b, L.w1);
        linear(c, L.w1, h2, ff_, I_, T, 2);  // gelu tanh (Gelu::Tanh, forward_gelu)
        linear(c, L.w2, x_, H, ff_, I_, T, 0, 1);
    }

    // post-LayerNorm, pixel shuffle, modality projection (:170-201)
    launch_layernorm(h_, x_, post_s_, post_b_, T, H, eps_, st);
    launch_pixel_shuffle(shuf_, h_, side_, H, sf_, st);
    linear(c, mm_, out_, mm_out_, shuf_, H * sf_ * sf_, ntok_);
}

void SiglipTf::encode_dev(const float* pixels, float* out, hipStream_t caller) {
    VLA_REQUIRE(pixels && out, "siglip: null buffer");
    launch_extract_patches(patches_, pixels, img_, P_, caller);
    replay_.run(1, own_, caller, [this](hipStream_t st) { run(st); });
    copy_f32(out, out_, (int64_t)ntok_ * mm_out_, caller);
}

}  // namespace hip
}  // namespace vla
