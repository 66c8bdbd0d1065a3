// model_act_full.cpp - ACT end to end on the device (see models.h).
//
// Follows src/models/act/act_model.cpp (config.txt, stats.bin, the camera and
// state normalization, the action un-normalization) and
// src/models/act/resnet_backbone.cpp (backbone.meta / .bin, the trunk). The
// fp32 convolutions are im2col + the fp32 matrix-core linear (their values
// differ from the reference's packed-panel GEMM only by summation order); the
// int8 ones are conv2d_i8, bit-exact to the reference's given the same input.
#include "ckpt.h"
#include "models.h"

#include <climits>
#include <cmath>
#include <cstdlib>
#include <sstream>

namespace vla {
namespace hip {

namespace {

// resnet_backbone.cpp:23-27
int conv_out(int in, int k, int stride, int pad) {
    const long long num = (long long)in + 2LL * pad - k;
    if (in <= 0 || stride <= 0 || num < 0 || num / stride >= INT_MAX) return 0;
    return (int)(num / stride + 1);
}

// arena.h shape_fits: every dim positive and the product within int
bool shape_fits(std::initializer_list<int> dims) {
    int count = 1;
    for (int d : dims) {
        if (d <= 0 || count > INT_MAX / d) return false;
        count *= d;
    }
    return true;
}

// hal::env::int_env (src/hal/common/env.cpp:23-29): a whole decimal integer,
// else the default
int int_env(const char* name, int dflt) {
    const char* e = std::getenv(name);
    if (!e || !*e) return dflt;
    char* end = nullptr;
    const long long v = std::strtoll(e, &end, 10);
    return *end || v < INT_MIN || v > INT_MAX ? dflt : (int)v;
}

// The values after a key, read as the reference's loaders read them: each
// `ss >> v` must succeed and nothing but whitespace may follow the last one.
template <class... T>
void read_values(const std::string& file, const std::string& key, const std::string& text, T&... v) {
    std::istringstream ss(text);
    (ss >> ... >> v);
    VLA_REQUIRE(!ss.fail() && (ss >> std::ws).eof(), file + ": bad value for key " + key + ": '" + text + "'");
}

struct Floats {
    const float* p;
    size_t n, off = 0;
    const float* take(size_t k, const char* what) {
        if (k > n - off) throw ArgError(std::string(what) + " is shorter than its .meta says");
        const float* r = p + off;
        off += k;
        return r;
    }
};

}  // namespace

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

    // <backbone>.meta (resnet_backbone.cpp:49-96): backbone.meta for ACT,
    // vision.meta for IMPACT
    const std::string bmeta = std::string(spec.backbone) + ".meta", bbin = std::string(spec.backbone) + ".bin";
    int in_ch = 3, stem_out = 64, stem_k = 7, stem_stride = 2, stem_pad = 3, gs = 0;
    struct BlockMeta {
        int cin, cout, stride, has_down;
    };
    std::vector<BlockMeta> bm;
    std::vector<int> film_after;
    for (const auto& kv : files.meta_lines(bmeta)) {
        const std::string& k = kv.first;
        const char* f = bmeta.c_str();
        if (k == "in_ch") read_values(f, k, kv.second, in_ch);
        else if (k == "stem_out") read_values(f, k, kv.second, stem_out);
        else if (k == "stem_k") read_values(f, k, kv.second, stem_k);
        else if (k == "stem_stride") read_values(f, k, kv.second, stem_stride);
        else if (k == "stem_pad") read_values(f, k, kv.second, stem_pad);
        else if (k == "pool_k") read_values(f, k, kv.second, pool_k_);
        else if (k == "pool_stride") read_values(f, k, kv.second, pool_stride_);
        else if (k == "pool_pad") read_values(f, k, kv.second, pool_pad_);
        else if (k == "gn_group_size") read_values(f, k, kv.second, gs);
        else if (k == "block") {
            BlockMeta b{};
            read_values(f, k, kv.second, b.cin, b.cout, b.stride, b.has_down);
            bm.push_back(b);
        } else if (k == "film_after") {
            int idx = -1;
            read_values(f, k, kv.second, idx);
            film_after.push_back(idx);
        }
    }
    const int bk = 3;
    VLA_REQUIRE(in_ch == 3 && shape_fits({stem_out, stem_k, stem_k, in_ch}) && stem_stride >= 1 && stem_pad >= 0 &&
                    stem_pad <= INT_MAX / 2 && pool_k_ >= 1 && pool_stride_ >= 1 && pool_pad_ >= 0 &&
                    pool_pad_ <= INT_MAX / 2 && gs >= 0,
                bmeta + ": invalid stem or pool (resnet_backbone.cpp:87-90 bounds)");
    VLA_REQUIRE(gs == 0, bmeta + ": group-norm trunks (gn_group_size > 0) are not supported on the device");
    for (const BlockMeta& b : bm)
        VLA_REQUIRE(shape_fits({b.cout, bk, bk, b.cin}) && shape_fits({b.cout, bk, bk, b.cout}) && b.stride >= 1 &&
                        (b.has_down == 0 || b.has_down == 1),
                    bmeta + ": invalid block (resnet_backbone.cpp:91-94 bounds)");

    // backbone.bin: stem, then per block conv1, conv2, down (:96-154). BatchNorm
    // is folded, so every conv carries a bias.
    const std::vector<char> raw = files.bytes(bbin);
    VLA_REQUIRE(raw.size() % 4 == 0, bbin + ": size is not a whole number of floats");
    Floats take{reinterpret_cast<const float*>(raw.data()), raw.size() / 4};
    // host copies of the fp32 weights for the int8 quantizer
    struct HostConv {
        const float *W, *b;
    };
    auto load_conv = [&](Conv& c, int cout, int k, int cin, int stride, int pad) {
        c.cout = cout;
        c.k = k;
        c.cin = cin;
        c.stride = stride;
        c.pad = pad;
        const float* W = take.take((size_t)cout * k * k * cin, bbin.c_str());
        const float* b = take.take(cout, bbin.c_str());
        c.W = A_.upload(W, (size_t)cout * k * k * cin);
        c.b = A_.upload(b, cout);
        return HostConv{W, b};
    };
    std::vector<HostConv> host;  // stem, then per block conv1, conv2, down
    host.push_back(load_conv(stem_, stem_out, stem_k, in_ch, stem_stride, stem_pad));
    blocks_.resize(bm.size());
    for (size_t i = 0; i < bm.size(); i++) {
        Block& blk = blocks_[i];
        const BlockMeta& m = bm[i];
        const int prev = i ? bm[i - 1].cout : stem_out;
        VLA_REQUIRE(m.cin == prev && m.cout >= 1 && m.stride >= 1,
                    bmeta + ": a block's input channels differ from the previous output");
        VLA_REQUIRE(m.has_down || (m.stride == 1 && m.cin == m.cout),
                    bmeta + ": a block without downsample changes shape");
        blk.has_down = m.has_down != 0;
        host.push_back(load_conv(blk.c1, m.cout, bk, m.cin, m.stride, 1));
        host.push_back(load_conv(blk.c2, m.cout, bk, m.cout, 1, 1));
        if (blk.has_down) host.push_back(load_conv(blk.down, m.cout, 1, m.cin, m.stride, 0));
    }
    VLA_REQUIRE(take.off == take.n, bbin + ": size does not match " + bmeta);
    int prev_idx = -1;
    for (int idx : film_after) {
        VLA_REQUIRE(idx >= 0 && idx < (int)blocks_.size() && idx > prev_idx,
                    bmeta + ": film_after must name blocks in ascending order");
        prev_idx = idx;
    }
    // FiLM points (film_total, resnet_backbone.cpp:190-195): block film_after[i]
    // reads gamma / beta at the sum of the earlier points' channels. ACT runs
    // its trunk unmodulated whatever the meta lists (act_model.cpp passes no
    // gamma / beta).
    film_off_.assign(blocks_.size(), -1);
    if (spec.film)
        for (int idx : film_after) {
            film_off_[idx] = film_total_;
            film_total_ += blocks_[idx].c1.cout;
        }

    // feature grid (ResNetBackbone::feat_size, :197-209)
    int h = conv_out(img_h_, stem_k, stem_stride, stem_pad), w = conv_out(img_w_, stem_k, stem_stride, stem_pad);
    const int h1 = h, w1 = w;
    h = conv_out(h, pool_k_, pool_stride_, pool_pad_);
    w = conv_out(w, pool_k_, pool_stride_, pool_pad_);
    const int ph = h, pw = w;
    size_t map_max = (size_t)h1 * w1 * stem_out, col_max = 0;
    map_max = std::max(map_max, (size_t)ph * pw * stem_out);
    // the im2col rows, then (64-float aligned) the split-K sums of the GEMM
    auto col_need = [&](const Conv& c, int H, int W) {
        const int Ho = conv_out(H, c.k, c.stride, c.pad), Wo = conv_out(W, c.k, c.stride, c.pad);
        const size_t npix = (size_t)Ho * Wo, K = (size_t)c.k * c.k * c.cin;
        const size_t rows = c.k == 1 && c.stride == 1 && c.pad == 0 ? 0 : col_rows_floats(npix, (int)K);
        col_max = std::max(col_max, rows + linear_f32_split_floats(Ho * Wo, c.cout, (int)K));
    };
    col_need(stem_, img_h_, img_w_);
    for (const Block& blk : blocks_) {
        const int oh = conv_out(h, bk, blk.c1.stride, 1), ow = conv_out(w, bk, blk.c1.stride, 1);
        col_need(blk.c1, h, w);
        col_need(blk.c2, oh, ow);
        if (blk.has_down) col_need(blk.down, h, w);
        map_max = std::max(map_max, (size_t)oh * ow * blk.c1.cout);
        h = oh;
        w = ow;
    }
    fh_ = h;
    fw_ = w;
    feat_ch_ = blocks_.empty() ? stem_out : blocks_.back().c1.cout;
    VLA_REQUIRE(shape_fits({fh_, fw_, feat_ch_, n_cams_}), "act: the backbone leaves no feature grid");

    // ACT_INT8 (act_model.cpp:57-64): bit 32 quantizes the convs of stages
    // [ACT_I8_CONV_FROM, ACT_I8_CONV_TO); Conv2d::init_int8 keeps a conv fp32
    // unless Cout % 16 == 0 and K is within the int8 bound (nn/conv.cpp:41-43)
    const int i8 = int_env(spec.int8_env, 0);
    if (i8 & 32) {
        const int from = int_env(spec.conv_from_env, 0);
        int to = int_env(spec.conv_to_env, -1);
        if (to < 0) to = (int)blocks_.size() + 1;
        auto want = [&](int stage) { return stage >= from && stage < to; };
        auto quantize = [&](Conv& c, const HostConv& hc) {
            const int K = c.k * c.k * c.cin;
            if (c.cout % 16 || K > kMaxI8K) return;
            c.q8 = vla_linear_i8::from_f32(hc.W, hc.b, c.cout, K);
            n_int8_convs_++;
        };
        size_t hi = 0;
        if (want(0)) quantize(stem_, host[0]);
        hi = 1;
        for (size_t i = 0; i < blocks_.size(); i++) {
            Block& blk = blocks_[i];
            const bool on = want((int)i + 1);
            if (on) quantize(blk.c1, host[hi]);
            if (on) quantize(blk.c2, host[hi + 1]);
            if (on && blk.has_down) quantize(blk.down, host[hi + 2]);
            hi += blk.has_down ? 3 : 2;
        }
    }
    tf_ = std::make_unique<ActTf>(dir, feat_ch_, i8, spec.int8_state, spec.tf);

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
    img_in_ = A_.alloc<uint8_t>((size_t)n_cams_ * npx * 3);
    norm_ = A_.alloc<float>((size_t)n_cams_ * npx * 3);
    part_norm_ = A_.alloc<float>((size_t)n_cams_ * kConvPartMax);
    part_a_ = A_.alloc<float>(kConvPartMax);
    part_b_ = A_.alloc<float>(kConvPartMax);
    part_c_ = A_.alloc<float>(kConvPartMax);
    a_ = A_.alloc<float>(map_max);
    b_ = A_.alloc<float>(map_max);
    c_ = A_.alloc<float>(map_max);
    res_ = A_.alloc<float>(map_max);
    col_ = A_.alloc<float>(col_max ? col_max : 4);
    col_floats_ = col_max;
    feats_ = A_.alloc<float>((size_t)n_cams_ * fh_ * fw_ * feat_ch_);
    state_n_ = A_.alloc<float>(sd);
    act_n_ = A_.alloc<float>((size_t)tf_->chunk() * ad);
    if (film_total_) {
        film_g_ = A_.alloc<float>(film_total_);
        film_b_ = A_.alloc<float>(film_total_);
    }
    if (n_int8_convs_) {
        size_t need = 0;
        auto ws = [&](const Conv& c, int H, int W) {
            if (c.q8) need = std::max(need, conv_shape(H, W, c.cin, c.k, c.stride, c.pad, c.cout).work);
        };
        h = img_h_;
        w = img_w_;
        ws(stem_, h, w);
        h = ph;
        w = pw;
        for (const Block& blk : blocks_) {
            const int oh = conv_out(h, bk, blk.c1.stride, 1), ow = conv_out(w, bk, blk.c1.stride, 1);
            ws(blk.c1, h, w);
            ws(blk.c2, oh, ow);
            if (blk.has_down) ws(blk.down, h, w);
            h = oh;
            w = ow;
        }
        work_bytes_ = need;
        work_ = A_.raw(need);
    }
    VLA_HIP_CHECK(hipStreamCreateWithFlags(&own_, hipStreamNonBlocking));
}

ActModel::~ActModel() {
    if (own_) (void)hipStreamDestroy(own_);
}

int ActModel::conv(const Conv& c, const float* x, int H, int W, float* out, bool relu, hipStream_t st,
                   const float* in_part, int in_nparts, float* out_part) {
    const int Ho = conv_out(H, c.k, c.stride, c.pad), Wo = conv_out(W, c.k, c.stride, c.pad);
    if (c.q8) {
        ConvArgs a{};
        a.out = out;
        a.x = x;
        a.Wq = c.q8->Wq();
        a.ldw = c.q8->ldw();
        a.wscale = c.q8->wscale();
        a.bias = c.q8->bias();
        a.H = H;
        a.Wd = W;
        a.Cin = c.cin;
        a.Cout = c.cout;
        a.k = c.k;
        a.stride = c.stride;
        a.pad = c.pad;
        a.clip = 0.0f;  // TCPU_I8_CLIP from the environment, as conv2d_i8 reads it
        a.work = work_;
        a.work_bytes = work_bytes_;
        // an fp32 producer (or none) wrote no maxima: conv2d_i8 runs its absmax pass
        a.in_part = in_nparts > 0 ? in_part : nullptr;
        a.in_nparts = in_nparts > 0 ? in_nparts : 0;
        launch_conv2d_i8(a, st);
        // the relu pass writes the block maxima the next conv2d_i8 reads
        return relu ? launch_relu_inplace(out, (int64_t)Ho * Wo * c.cout, st, out_part) : 0;
    }
    const int K = c.k * c.k * c.cin;
    const float* rows = x;
    int ldx = K;
    const bool plain = c.k == 1 && c.stride == 1 && c.pad == 0;  // the map is already the GEMM's A
    // split-K sums after the im2col rows (the implicit form leaves those unused)
    const size_t rows_f = plain ? 0 : col_rows_floats((size_t)Ho * Wo, K);
    float* part = col_ + rows_f;
    const size_t part_f = col_floats_ - rows_f;
    if (!plain && launch_conv_f32_implicit(out, x, H, W, c.cin, c.k, c.stride, c.pad, Ho, Wo, c.W, c.b, c.cout,
                                           relu ? 1 : 0, st, part, part_f))
        return 0;
    if (!plain) {
        ldx = (K + 3) & ~3;
        launch_im2col_f32(col_, ldx, x, H, W, c.cin, c.k, c.stride, c.pad, Ho, Wo, st);
        rows = col_;
    }
    launch_linear_f32(out, c.cout, rows, ldx, c.W, K, c.b, Ho * Wo, c.cout, K, relu ? 1 : 0, 0, 1.0f, st, part,
                      part_f);
    return 0;
}

// ActModel::encode_view for every camera (act_model.cpp:106-124) and
// ResNetBackbone::forward (resnet_backbone.cpp:211-317); FiLM at the points
// film_off_ names (IMPACT)
//
// With int8 convolutions each conv2d_i8 input comes with the block maxima of
// |x| that its producer wrote (the normalization, the max pool, the relu
// after conv1, the block's residual add + relu), so no conv runs an absmax
// pass of its own; the maxima buffers follow the trunk buffers they describe.
void ActModel::run_backbone(hipStream_t st) {
    const int64_t npx = (int64_t)img_h_ * img_w_;
    const int nn = launch_normalize_u8(norm_, img_in_, n_cams_, npx, img_mean_, img_std_, norm_eps_, st,
                                       stem_.q8 ? part_norm_ : nullptr);
    for (int cam = 0; cam < n_cams_; cam++) {
        const float* x = norm_ + (size_t)cam * npx * 3;
        int h = conv_out(img_h_, stem_.k, stem_.stride, stem_.pad), w = conv_out(img_w_, stem_.k, stem_.stride, stem_.pad);
        conv(stem_, x, img_h_, img_w_, a_, false, st, part_norm_ + (size_t)cam * kConvPartMax, nn);
        const int ph = conv_out(h, pool_k_, pool_stride_, pool_pad_), pw = conv_out(w, pool_k_, pool_stride_, pool_pad_);
        float* B = b_;
        float* C = c_;
        float* pB = part_b_;
        float* pC = part_c_;
        int nB = launch_maxpool_relu(B, a_, h, w, stem_.cout, pool_k_, pool_stride_, pool_pad_, ph, pw, st, pB);
        h = ph;
        w = pw;
        for (size_t bi = 0; bi < blocks_.size(); bi++) {
            const Block& blk = blocks_[bi];
            const int oh = conv_out(h, blk.c1.k, blk.c1.stride, blk.c1.pad);
            const int ow = conv_out(w, blk.c1.k, blk.c1.stride, blk.c1.pad);
            const float* idn = B;
            if (blk.has_down) {
                conv(blk.down, B, h, w, res_, false, st, pB, nB);
                idn = res_;
            }
            const int nA = conv(blk.c1, B, h, w, a_, true, st, pB, nB, part_a_);
            conv(blk.c2, a_, oh, ow, C, false, st, part_a_, nA);
            const int64_t n = (int64_t)oh * ow * blk.c1.cout;
            const int fo = film_off_[bi];
            nB = fo >= 0 ? launch_add_relu_film(C, idn, n, blk.c1.cout, film_g_ + fo, film_b_ + fo, st, pC)
                         : launch_add_relu(C, idn, n, st, pC);
            std::swap(B, C);
            std::swap(pB, pC);
            h = oh;
            w = ow;
        }
        copy_f32(feats_ + (size_t)cam * fh_ * fw_ * feat_ch_, B, (int64_t)fh_ * fw_ * feat_ch_, st);
    }
}

void ActModel::encode_dev(const uint8_t* images, float* feats, hipStream_t caller) {
    VLA_REQUIRE(images && feats, "act: null buffer");
    VLA_HIP_CHECK(hipMemcpyAsync(img_in_, images, (size_t)n_cams_ * img_h_ * img_w_ * 3, hipMemcpyDeviceToDevice,
                                 caller));
    replay_.run(1, own_, caller, [this](hipStream_t st) { run_backbone(st); });
    copy_f32(feats, feats_, (int64_t)n_cams_ * fh_ * fw_ * feat_ch_, caller);
}

// ActModel::predict (act_model.cpp:126-164), ImpactModel::predict
// (impact_model.cpp:201-244) with the text tail
void ActModel::predict_text_dev(const uint8_t* images, const float* state, const float* text, const float* text_pos,
                                int n_text_real, bool unnormalize, float* actions, hipStream_t caller) {
    VLA_REQUIRE(images && state && actions, "act: null buffer");
    VLA_HIP_CHECK(hipMemcpyAsync(img_in_, images, (size_t)n_cams_ * img_h_ * img_w_ * 3, hipMemcpyDeviceToDevice,
                                 caller));
    replay_.run(1, own_, caller, [this](hipStream_t st) { run_backbone(st); });
    launch_col_affine(state_n_, state, 1, tf_->state_dim(), state_mean_, state_std_, norm_eps_, 0, caller);
    const int C = tf_->chunk(), ad = tf_->action_dim();
    tf_->forward_text_dev(feats_, n_cams_, fh_, fw_, state_n_, text, text_pos, n_text_real,
                          unnormalize ? act_n_ : actions, caller);
    if (unnormalize) launch_col_affine(actions, act_n_, C, ad, action_mean_, action_std_, 0.0f, 1, caller);
}

}  // namespace hip
}  // namespace vla
