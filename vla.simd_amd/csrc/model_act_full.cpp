// model_act_full.cpp - ACT end to end on the device (see models.h).
//
// Follows src/models/act/act_model.cpp (config.txt, stats.bin, the camera and
// state normalization, the action un-normalization); the trunk
// (resnet_backbone.cpp) is ResNetTrunk (resnet.cpp).
#include "ckpt.h"
#include "loader.h"
#include "models.h"

#include <cmath>

namespace vla {
namespace hip {

ActModel::ActModel(const std::string& dir, const ActSpec& spec) {
    const CkptFiles files(dir);

    // config.txt (act_model.cpp:24-45)
    for (const auto& kv : files.meta_lines("config.txt")) {
        const std::string& k = kv.first;
        if (k == "img_h") read_values("config.txt", k, kv.second, img_h_);
        else if (k == "img_w") read_values("config.txt", k, kv.second, img_w_);
        else if (k == "n_cams") read_values("config.txt", k, kv.second, n_cams_);
        else if (k == "norm_eps") read_values("config.txt", k, kv.second, norm_eps_);
        else if (k.rfind("cam", 0) == 0) {
            std::string name;
            read_values("config.txt", k, kv.second, name);
        }
    }
    VLA_REQUIRE(shape_fits({img_h_, img_w_, n_cams_, 3}) && std::isfinite(norm_eps_) && norm_eps_ > 0,
                "config.txt: invalid image shape or norm_eps (act_model.cpp:46-47 bounds)");

    // the trunk: <backbone>.meta / .bin (backbone.* for ACT, vision.* for
    // IMPACT). ACT_INT8 (act_model.cpp:57-64): bit 32 quantizes the convs of
    // stages [ACT_I8_CONV_FROM, ACT_I8_CONV_TO).
    const int i8 = int_env(spec.int8_env, 0);
    TrunkOpts to;
    to.film = spec.film;
    to.int8 = (i8 & 32) != 0;
    to.from = int_env(spec.conv_from_env, 0);
    to.to = int_env(spec.conv_to_env, -1);
    trunk_ = std::make_unique<ResNetTrunk>(files, spec.backbone, img_h_, img_w_, to);
    const int fh = trunk_->feat_h(), fw = trunk_->feat_w(), feat_ch = trunk_->channels();
    VLA_REQUIRE(shape_fits({fh, fw, feat_ch, n_cams_}), "act: the backbone leaves no feature grid");
    tf_ = std::make_unique<ActTf>(dir, feat_ch, i8, spec.int8_state, spec.tf);

    // stats.bin (act_model.cpp:66-101)
    const int sd = tf_->state_dim(), ad = tf_->action_dim();
    const std::vector<char> st = files.bytes("stats.bin");
    const size_t nstat = (size_t)2 * sd + 2 * ad + (size_t)n_cams_ * 6;
    VLA_REQUIRE(st.size() == nstat * 4, "stats.bin: size does not match the state, action and camera counts");
    const float* p = reinterpret_cast<const float*>(st.data());
    for (size_t i = 0; i < nstat; i++) VLA_REQUIRE(std::isfinite(p[i]), "stats.bin: non-finite value");
    std::vector<float> im((size_t)n_cams_ * 3), is((size_t)n_cams_ * 3);
    for (int c = 0; c < n_cams_; c++)
        for (int i = 0; i < 3; i++) {
            im[(size_t)c * 3 + i] = p[2 * sd + 2 * ad + (size_t)c * 6 + i];
            is[(size_t)c * 3 + i] = p[2 * sd + 2 * ad + (size_t)c * 6 + 3 + i];
        }
    auto nonneg = [](const float* v, size_t n) {
        for (size_t i = 0; i < n; i++)
            if (v[i] < 0) return false;
        return true;
    };
    VLA_REQUIRE(nonneg(p + sd, sd) && nonneg(p + 2 * sd + ad, ad) && nonneg(is.data(), is.size()),
                "stats.bin: negative standard deviation");
    state_mean_ = A_.upload(p, sd);
    state_std_ = A_.upload(p + sd, sd);
    action_mean_ = A_.upload(p + 2 * sd, ad);
    action_std_ = A_.upload(p + 2 * sd + ad, ad);
    img_mean_ = A_.upload(im.data(), im.size());
    img_std_ = A_.upload(is.data(), is.size());

    // buffers
    const size_t npx = (size_t)img_h_ * img_w_;
    norm_ = A_.alloc<float>((size_t)n_cams_ * npx * 3);
    part_norm_ = A_.alloc<float>((size_t)n_cams_ * kConvPartMax);
    feats_ = A_.alloc<float>((size_t)n_cams_ * fh * fw * feat_ch);
    state_n_ = A_.alloc<float>(sd);
    act_n_ = A_.alloc<float>((size_t)tf_->chunk() * ad);
    VLA_HIP_CHECK(hipStreamCreateWithFlags(&own_, hipStreamNonBlocking));
}

ActModel::~ActModel() {
    if (own_) (void)hipStreamDestroy(own_);
}

// ActModel::encode_view for every camera (act_model.cpp:106-124): the
// normalization (with the block maxima an int8 stem reads), then the trunk
void ActModel::run_backbone(hipStream_t st, const uint8_t* images, float* feats) {
    const int64_t npx = (int64_t)img_h_ * img_w_;
    const bool q = trunk_->stem_int8();
    const int nn = launch_normalize_u8(norm_, images, n_cams_, npx, img_mean_, img_std_, norm_eps_, st,
                                       q ? part_norm_ : nullptr);
    const size_t nf = (size_t)trunk_->feat_h() * trunk_->feat_w() * trunk_->channels();
    for (int cam = 0; cam < n_cams_; cam++)
        trunk_->run(norm_ + (size_t)cam * npx * 3, part_norm_ + (size_t)cam * kConvPartMax, nn, feats + cam * nf,
                    st);
}

void ActModel::encode_dev(const uint8_t* images, float* feats, hipStream_t caller) {
    VLA_REQUIRE(images && feats, "act: null buffer");
    if (images != enc_img_ || feats != enc_feats_) {
        enc_img_ = images;
        enc_feats_ = feats;
        enc_key_++;
    }
    enc_replay_.run(enc_key_, own_, caller, [this, images, feats](hipStream_t st) { run_backbone(st, images, feats); });
}

// ActModel::predict (act_model.cpp:126-164), ImpactModel::predict
// (impact_model.cpp:201-244) with the text tail
void ActModel::predict_text_dev(const uint8_t* images, const float* state, const float* text, const float* text_pos,
                                int n_text_real, bool unnormalize, float* actions, hipStream_t caller) {
    VLA_REQUIRE(images && state && actions, "act: null buffer");
    if (images != pred_img_) {
        pred_img_ = images;
        pred_key_++;
    }
    replay_.run(pred_key_, own_, caller, [this, images](hipStream_t st) { run_backbone(st, images, feats_); });
    launch_col_affine(state_n_, state, 1, tf_->state_dim(), state_mean_, state_std_, norm_eps_, 0, caller);
    const int C = tf_->chunk(), ad = tf_->action_dim();
    tf_->forward_text_dev(feats_, n_cams_, feat_h(), feat_w(), state_n_, text, text_pos, n_text_real,
                          unnormalize ? act_n_ : actions, caller);
    if (unnormalize) launch_col_affine(actions, act_n_, C, ad, action_mean_, action_std_, 0.0f, 1, caller);
}

}  // namespace hip
}  // namespace vla
