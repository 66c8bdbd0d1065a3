// model_octo_full.cpp - Octo end to end on the device (see models.h).
//
// Follows src/models/octo/octo_model.cpp (load, the OCTO_INT8 groups, the
// instruction cache, the stem window reuse, the DDPM noise draw, the
// un-normalization), octo_capi.cpp (the argument checks), small_stem.cpp,
// diffusion_head.cpp + src/nn/diffusion.cpp, and src/nn/t5_encoder.cpp. The
// block transformer is OctoTf. Every op runs on the device on one stream; the
// host tokenizes, builds the T5 bias table once per instruction and compares
// frames for the stem reuse.
#include "ckpt.h"
#include "models.h"

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <random>
#include <sstream>

namespace vla {
namespace hip {

namespace {

// arena.h metadata_int: a finite whole number within int
int whole(const std::string& file, const std::string& key, double v) {
    VLA_REQUIRE(std::isfinite(v) && v == std::trunc(v) && v >= -2147483648.0 && v <= 2147483647.0,
                file + ": " + key + " is not an integer");
    return (int)v;
}

bool fits(std::initializer_list<int> dims) {
    int count = 1;
    for (int d : dims) {
        if (d <= 0 || count > INT_MAX / d) return false;
        count *= d;
    }
    return true;
}

// "key value" pairs, every value a finite number (the `meta >> key >> val`
// loops of t5_encoder.cpp:22-35 and diffusion_head.cpp:19-32)
std::vector<std::pair<std::string, double>> kv_pairs(const CkptFiles& files, const std::string& rel) {
    const std::vector<char> b = files.bytes(rel);
    std::istringstream in(std::string(b.begin(), b.end()));
    std::vector<std::pair<std::string, double>> out;
    std::string k;
    double v;
    while (in >> k) {
        VLA_REQUIRE(static_cast<bool>(in >> v) && std::isfinite(v), rel + ": bad value for key " + k);
        out.emplace_back(k, v);
    }
    return out;
}

// read_arena + ArenaCursor (arena.h:44-72): a .bin of whole floats taken in order
struct Arena {
    std::vector<float> d;
    size_t off = 0;
    std::string what;
    Arena(const CkptFiles& files, const std::string& rel) : what(rel) {
        const std::vector<char> b = files.bytes(rel);
        VLA_REQUIRE(b.size() % 4 == 0, rel + ": size is not a whole number of floats");
        d.resize(b.size() / 4);
        std::memcpy(d.data(), b.data(), b.size());
    }
    const float* take(size_t n) {
        VLA_REQUIRE(n <= d.size() - off, what + " is shorter than its .meta says");
        const float* p = d.data() + off;
        off += n;
        return p;
    }
    void done() const { VLA_REQUIRE(off == d.size(), what + ": size does not match its .meta"); }
};

int env_int(const char* name, int dflt) {
    const char* e = std::getenv(name);
    if (!e || !*e) return dflt;
    char* end = nullptr;
    const long long v = std::strtoll(e, &end, 10);
    return *end || v < INT_MIN || v > INT_MAX ? dflt : (int)v;
}

// nn::Linear::init_int8 / Conv2d::init_int8 take a layer only when N % 16 == 0
// and K is within the int8 bound (linear.cpp:67-68, conv.cpp:40-43)
bool int8_fits(int N, int K) { return N % 16 == 0 && K > 0 && K <= kMaxI8K; }

// HF T5 _relative_position_bucket, bidirectional, rp = key - query
// (t5_encoder.cpp:66-79)
int rel_bucket(int rp, int num_buckets, int max_dist) {
    const int nb = num_buckets / 2;
    const int base = rp > 0 ? nb : 0;
    const int a = rp < 0 ? -rp : rp;
    const int exact = nb / 2;
    if (a < exact) return base + a;
    int large = exact + (int)(std::log((double)a / exact) / std::log((double)max_dist / exact) * (nb - exact));
    if (large > nb - 1) large = nb - 1;
    return base + large;
}

}  // namespace

// ------------------------------------------------------------------- T5 --

T5Enc::T5Enc(const CkptFiles& files, const std::string& stem, std::vector<float>* tail) {
    const std::string mf = stem + ".meta";
    for (const auto& kv : kv_pairs(files, mf)) {
        const std::string& k = kv.first;
        if (k == "d_model") D_ = whole(mf, k, kv.second);
        else if (k == "n_layers") NL_ = whole(mf, k, kv.second);
        else if (k == "n_heads") NH_ = whole(mf, k, kv.second);
        else if (k == "d_kv") HD_ = whole(mf, k, kv.second);
        else if (k == "d_ff") FF_ = whole(mf, k, kv.second);
        else if (k == "vocab") vocab_ = whole(mf, k, kv.second);
        else if (k == "n_buckets") nb_ = whole(mf, k, kv.second);
        else if (k == "max_dist") maxd_ = whole(mf, k, kv.second);
        else if (k == "eps") eps_ = (float)kv.second;
    }
    VLA_REQUIRE(fits({D_, D_}) && fits({D_, FF_}) && fits({vocab_, D_}) && fits({NH_, HD_}) && NH_ * HD_ == D_ &&
                    NL_ >= 1 && fits({nb_, NH_}) && nb_ >= 4 && nb_ % 2 == 0 && maxd_ > nb_ / 4 &&
                    std::isfinite(eps_) && eps_ > 0,
                mf + ": shapes do not close (t5_encoder.cpp:36-40 bounds)");
    Arena a(files, stem + ".bin");
    const int D = D_, FF = FF_;
    emb_ = A_.upload(a.take((size_t)vocab_ * D), (size_t)vocab_ * D);
    const float* rel = a.take((size_t)nb_ * NH_);
    rel_.assign(rel, rel + (size_t)nb_ * NH_);
    layers_.resize(NL_);
    std::vector<float> qkv((size_t)3 * D * D);
    for (Layer& L : layers_) {
        L.ln1 = A_.upload(a.take(D), D);
        for (int i = 0; i < 3; i++) std::memcpy(qkv.data() + (size_t)i * D * D, a.take((size_t)D * D), (size_t)D * D * 4);
        L.wqkv = A_.upload(qkv.data(), qkv.size());
        L.wo = A_.upload(a.take((size_t)D * D), (size_t)D * D);
        L.ln2 = A_.upload(a.take(D), D);
        L.wi = A_.upload(a.take((size_t)FF * D), (size_t)FF * D);
        L.wo2 = A_.upload(a.take((size_t)D * FF), (size_t)D * FF);
    }
    final_ = A_.upload(a.take(D), D);
    if (tail)  // T5Encoder::load's enc_end: what follows belongs to the caller
        tail->assign(a.d.begin() + (std::ptrdiff_t)a.off, a.d.end());
    else
        a.done();
}

// T5Encoder::encode (t5_encoder.cpp:81-134)
void T5Enc::encode_dev(const int32_t* ids, const int32_t* mask, int seq, float* out, hipStream_t st) {
    VLA_REQUIRE(seq > 0 && ids && mask && out, "t5: bad arguments");
    const int D = D_, NH = NH_, HD = HD_, FF = FF_;
    if (seq > seq_cap_) {
        VLA_HIP_CHECK(hipStreamSynchronize(st));
        S_ = std::make_unique<DeviceArena>();
        x_ = S_->alloc<float>((size_t)seq * D);
        h_ = S_->alloc<float>((size_t)seq * D);
        qkv_ = S_->alloc<float>((size_t)seq * 3 * D);
        att_ = S_->alloc<float>((size_t)seq * D);
        ff_ = S_->alloc<float>((size_t)seq * FF);
        bias_ = S_->alloc<float>((size_t)NH * seq * seq);
        ids_ = S_->alloc<int32_t>(seq);
        seq_cap_ = seq;
    }
    // per-head additive bias: the relative position bias, lowest() on padded keys
    const float NEG = std::numeric_limits<float>::lowest();
    std::vector<float> bias((size_t)NH * seq * seq);
    for (int h = 0; h < NH; h++)
        for (int i = 0; i < seq; i++)
            for (int j = 0; j < seq; j++)
                bias[((size_t)h * seq + i) * seq + j] =
                    mask[j] ? rel_[(size_t)rel_bucket(j - i, nb_, maxd_) * NH + h] : NEG;
    VLA_HIP_CHECK(hipMemcpyAsync(bias_, bias.data(), bias.size() * 4, hipMemcpyHostToDevice, st));
    VLA_HIP_CHECK(hipMemcpyAsync(ids_, ids, (size_t)seq * 4, hipMemcpyHostToDevice, st));
    launch_embed_f32(x_, emb_, ids_, seq, D, vocab_, st);
    for (const Layer& L : layers_) {
        launch_rmsnorm(h_, x_, L.ln1, seq, D, eps_, st);
        launch_linear_f32(qkv_, 3 * D, h_, D, L.wqkv, D, nullptr, seq, 3 * D, D, 0, 0, 1.0f, st);
        for (int h = 0; h < NH; h++) {  // attention with this head's bias, no 1/sqrt(d) scale
            MaskSpec m;
            m.kind = 1;
            m.dense = bias_ + (size_t)h * seq * seq;
            m.ldm = seq;
            attend(st, att_ + h * HD, D, qkv_ + h * HD, 3 * D, qkv_ + D + h * HD, 3 * D, qkv_ + 2 * D + h * HD,
                   3 * D, seq, seq, 1, 1, HD, 1.0f, m);
        }
        launch_linear_f32(x_, D, att_, D, L.wo, D, nullptr, seq, D, D, 0, 1, 1.0f, st);  // x += att Wo
        launch_rmsnorm(h_, x_, L.ln2, seq, D, eps_, st);
        launch_linear_f32(ff_, FF, h_, D, L.wi, D, nullptr, seq, FF, D, 1, 0, 1.0f, st);  // relu
        launch_linear_f32(x_, D, ff_, FF, L.wo2, FF, nullptr, seq, D, FF, 0, 1, 1.0f, st);
    }
    launch_rmsnorm(out, x_, final_, seq, D, eps_, st);
    // the host bias table and ids must outlive their copies; this runs once
    // per new instruction
    VLA_HIP_CHECK(hipStreamSynchronize(st));
}

// ----------------------------------------------------------- SmallStem --

OctoStem::OctoStem(const CkptFiles& files, const std::string& name, int int8_mask, int H, int W) : H_(H), W_(W) {
    // <name>.meta (small_stem.cpp:19-37): one key per line, the value(s) read
    // with >> and nothing after them
    int in_ch = 6, n_layers = 4;
    std::vector<int> features = {32, 96, 192, 384, 0, 0, 0, 0};
    const std::string mf = name + ".meta";
    for (const auto& kv : files.meta_lines(mf)) {
        const std::string& k = kv.first;
        std::istringstream ss(kv.second);
        if (k == "in_ch") ss >> in_ch;
        else if (k == "n_layers") ss >> n_layers;
        else if (k == "k") ss >> k_;
        else if (k == "stride") ss >> stride_;
        else if (k == "pad") ss >> pad_;
        else if (k == "features")
            for (int i = 0; i < n_layers && i < 8; i++) ss >> features[i];
        else if (k == "embed_dim") ss >> embed_dim_;
        else if (k == "gn_groups") ss >> groups_;
        else if (k == "gn_eps") ss >> gn_eps_;
        else continue;
        VLA_REQUIRE(!ss.fail() && (ss >> std::ws).eof(), mf + ": bad value for key " + k);
    }
    VLA_REQUIRE(n_layers >= 1 && n_layers <= 8 && in_ch == 6 && k_ >= 1 && embed_dim_ >= 1 && stride_ >= 1 &&
                    pad_ >= 0 && pad_ <= (INT_MAX - 256) / 2 && groups_ >= 1 && std::isfinite(gn_eps_) &&
                    gn_eps_ > 0,
                mf + ": invalid stem (small_stem.cpp:42-50 bounds)");
    int cin = in_ch;
    for (int i = 0; i < n_layers; i++) {
        VLA_REQUIRE(fits({features[i], k_, k_, cin}) && features[i] % groups_ == 0,
                    mf + ": invalid features (small_stem.cpp:51-54 bounds)");
        // the device GroupNorm's limits (launch_groupnorm), checked at load
        VLA_REQUIRE(features[i] <= 1024 && features[i] / groups_ <= 256,
                    mf + ": GroupNorm beyond this build (at most 1024 channels, 256 per group)");
        cin = features[i];
    }

    // <name>.bin: per layer conv W [cout, k, k, cin], b, gn scale, gn bias;
    // then the embedding [embed_dim, cin], b (:60-82)
    Arena a(files, name + ".bin");
    const bool conv8 = (int8_mask & 16) != 0, emb8 = (int8_mask & 8) != 0;
    cin = in_ch;
    int h = H, w = W;
    size_t act_max = (size_t)H * W * in_ch, col_max = 4, work = 0;
    layers_.resize(n_layers);
    for (int i = 0; i < n_layers; i++) {
        Layer& L = layers_[i];
        L.cin = cin;
        L.cout = features[i];
        L.H = h;
        L.W = w;
        const long long nh = (long long)h + 2LL * pad_ - k_, nw = (long long)w + 2LL * pad_ - k_;
        VLA_REQUIRE(nh >= 0 && nw >= 0, name + ": the image is smaller than the stem's kernel");
        L.Ho = (int)(nh / stride_ + 1);
        L.Wo = (int)(nw / stride_ + 1);
        const int K = k_ * k_ * cin;
        const float* Wt = a.take((size_t)L.cout * K);
        const float* b = a.take(L.cout);
        if (conv8 && int8_fits(L.cout, K)) {
            L.q8 = vla_linear_i8::from_f32(Wt, b, L.cout, K);
            n_int8_++;
            work = std::max(work, conv_shape(h, w, cin, k_, stride_, pad_, L.cout).work);
        } else {
            L.W_ = A_.upload(Wt, (size_t)L.cout * K);
            L.b = A_.upload(b, L.cout);
            // the im2col rows, then the GEMM's split-K sums
            col_max = std::max(col_max, col_rows_floats((size_t)L.Ho * L.Wo, K) +
                                            linear_f32_split_floats(L.Ho * L.Wo, L.cout, K));
        }
        L.gs = A_.upload(a.take(L.cout), L.cout);
        L.gb = A_.upload(a.take(L.cout), L.cout);
        act_max = std::max(act_max, (size_t)L.Ho * L.Wo * L.cout);
        cin = L.cout;
        h = L.Ho;
        w = L.Wo;
    }
    const float* ew = a.take((size_t)embed_dim_ * cin);
    const float* eb = a.take(embed_dim_);
    a.done();
    VLA_REQUIRE(fits({h, w}), name + ": no token grid");
    tok_ = h * w;
    const bool e8 = emb8 && int8_fits(embed_dim_, cin);
    embed_.init(A_, ew, eb, embed_dim_, cin, e8);
    n_int8_ += e8 ? 1 : 0;
    a_ = A_.alloc<float>(act_max);
    b_ = A_.alloc<float>(act_max);
    col_ = A_.alloc<float>(col_max);
    col_floats_ = col_max;
    int cmax = 1;
    for (const Layer& L : layers_) cmax = std::max(cmax, L.cout);
    gA_ = A_.alloc<float>(cmax);
    gB_ = A_.alloc<float>(cmax);
    for (const Layer& L : layers_) gw_doubles_ = std::max(gw_doubles_, groupnorm_work_doubles(L.Ho * L.Wo, L.cout));
    gW_ = A_.alloc<double>(gw_doubles_);
    if (work) {
        work_ = A_.raw(work);
        work_bytes_ = work;
    }
    ctx_.alloc(A_, tok_, round_up(kpad4(cin), 64));
}

// SmallStem::encode (small_stem.cpp:84-142)
void OctoStem::encode_dev(const uint8_t* img, float* out, hipStream_t st) {
    launch_stem_input(a_, img, (int64_t)H_ * W_, st);
    for (const Layer& L : layers_) {
        const int K = k_ * k_ * L.cin;
        if (L.q8) {
            ConvArgs c{};
            c.out = b_;
            c.x = a_;
            c.Wq = L.q8->Wq();
            c.ldw = L.q8->ldw();
            c.wscale = L.q8->wscale();
            c.bias = L.q8->bias();
            c.H = L.H;
            c.Wd = L.W;
            c.Cin = L.cin;
            c.Cout = L.cout;
            c.k = k_;
            c.stride = stride_;
            c.pad = pad_;
            c.clip = 0.0f;
            c.work = work_;
            c.work_bytes = work_bytes_;
            launch_conv2d_i8(c, st);
        } else {
            const size_t rows_f = col_rows_floats((size_t)L.Ho * L.Wo, K);
            float* part = col_ + rows_f;  // split-K sums after the im2col rows
            const size_t part_f = col_floats_ - rows_f;
            if (!launch_conv_f32_implicit(b_, a_, L.H, L.W, L.cin, k_, stride_, pad_, L.Ho, L.Wo, L.W_, L.b, L.cout,
                                          0, st, part, part_f)) {
                const int ldc = kpad4(K);
                launch_im2col_f32(col_, ldc, a_, L.H, L.W, L.cin, k_, stride_, pad_, L.Ho, L.Wo, st);
                launch_linear_f32(b_, L.cout, col_, ldc, L.W_, K, L.b, L.Ho * L.Wo, L.cout, K, 0, 0, 1.0f, st, part,
                                  part_f);
            }
        }
        launch_groupnorm(a_, b_, L.gs, L.gb, L.Ho * L.Wo, L.cout, groups_, gn_eps_, true, gA_, gB_, gW_, gw_doubles_,
                         st);
    }
    Ctx c = ctx_;
    c.st = st;
    linear(c, embed_, out, embed_dim_, a_, layers_.back().cout, tok_);
}

// ------------------------------------------------------------ DDPM head --

OctoHead::OctoHead(const CkptFiles& files, int int8_mask) {
    for (const auto& kv : kv_pairs(files, "head.meta")) {
        const std::string& k = kv.first;
        if (k == "emb") emb_ = whole("head.meta", k, kv.second);
        else if (k == "action_dim") ad_ = whole("head.meta", k, kv.second);
        else if (k == "horizon") horizon_ = whole("head.meta", k, kv.second);
        else if (k == "time_dim") td_ = whole("head.meta", k, kv.second);
        else if (k == "num_blocks") nb_ = whole("head.meta", k, kv.second);
        else if (k == "hidden") H_ = whole("head.meta", k, kv.second);
        else if (k == "steps") steps_ = whole("head.meta", k, kv.second);
        else if (k == "max_action") max_action_ = (float)kv.second;
    }
    const int FLAT = ad_ * horizon_;
    VLA_REQUIRE(fits({ad_, horizon_}) && fits({2, td_, td_}) && td_ % 2 == 0 && fits({4, H_, H_}) && emb_ >= 1 &&
                    nb_ >= 0 && (long long)td_ + emb_ + FLAT <= INT_MAX && fits({steps_, td_}) &&
                    std::isfinite(max_action_) && max_action_ > 0,
                "head.meta: invalid head (diffusion_head.cpp:34-40 bounds)");
    Arena a(files, "head.bin");
    const int TD = td_, H = H_, IN = TD + emb_ + FLAT;
    const bool i8 = (int8_mask & 32) != 0;
    auto lin = [&](DLinear& L, int N, int K, bool want8) {
        const float* w = a.take((size_t)N * K);
        const float* b = a.take(N);
        const bool q = want8 && int8_fits(N, K);
        L.init(A_, w, b, N, K, q);
        n_int8_ += q ? 1 : 0;
    };
    const float* fw = a.take(TD / 2);
    DLinear cond0, cond1;  // the time conditioning MLP: fp32, used once here
    lin(cond0, 2 * TD, TD, false);
    lin(cond1, TD, 2 * TD, false);
    lin(in_proj_, H, IN, i8);
    blocks_.resize(nb_);
    for (Block& B : blocks_) {
        B.ln_s = A_.upload(a.take(H), H);
        B.ln_b = A_.upload(a.take(H), H);
        lin(B.d0, 4 * H, H, i8);
        lin(B.d1, H, 4 * H, i8);
    }
    lin(out_proj_, FLAT, H, i8);
    const float* betas = a.take(steps_);
    const float* alphas = a.take(steps_);
    const float* ahat = a.take(steps_);
    a.done();
    for (int t = 0; t < steps_; t++)
        VLA_REQUIRE(betas[t] > 0 && betas[t] < 1 && alphas[t] > 0 && alphas[t] < 1 && ahat[t] > 0 && ahat[t] < 1 &&
                        (t == 0 || ahat[t] <= ahat[t - 1]),
                    "head.bin: invalid noise schedule (diffusion_head.cpp:112-117)");
    // per-step coefficients of the reverse update, in float as the reference
    a1_.resize(steps_);
    a2_.resize(steps_);
    sb_.resize(steps_);
    for (int t = 0; t < steps_; t++) {
        a1_[t] = 1.0f / std::sqrt(alphas[t]);
        a2_[t] = (1.0f - alphas[t]) / std::sqrt(1.0f - ahat[t]);
        sb_[t] = t > 0 ? std::sqrt(betas[t]) : 0.0f;
    }

    const int R = 4 * H > IN ? 4 * H : IN;
    in_ = A_.alloc<float>(IN);
    h_ = A_.alloc<float>(H);
    n_ = A_.alloc<float>(H);
    wide_ = A_.alloc<float>(4 * H);
    e_ = A_.alloc<float>(FLAT);
    ctx_.alloc(A_, 1, round_up(kpad4(R), 64));

    // the time conditioning of t = 0..steps-1 (diffusion_head.cpp:121-138):
    // Fourier features -> cond0 -> silu -> cond1
    cond_ = A_.alloc<float>((size_t)steps_ * TD);
    float* tff = A_.alloc<float>((size_t)steps_ * TD);
    float* c1 = A_.alloc<float>((size_t)steps_ * 2 * TD);
    float* wdev = A_.upload(fw, TD / 2);
    hipStream_t st = library_stream();
    Ctx c = ctx_;
    c.st = st;
    launch_fourier(tff, wdev, steps_, TD, st);
    linear(c, cond0, c1, 2 * TD, tff, TD, steps_, 4);  // silu
    linear(c, cond1, cond_, TD, c1, 2 * TD, steps_);

    // the fused form of denoise_dev: every layer's weights, the per-step
    // coefficients on the device; used when the shapes fit its one workgroup
    auto hl = [](const DLinear& L) {
        HeadLin h;
        if (L.int8()) {
            h.Wq = L.q8->Wq();
            h.ldw = L.q8->ldw();
            h.ws = L.q8->wscale();
            h.b = L.q8->bias();
        } else {
            h.W = L.W;
            h.b = L.b;
        }
        h.N = L.N;
        h.K = L.K;
        return h;
    };
    fused_.in_proj = hl(in_proj_);
    fused_.out_proj = hl(out_proj_);
    fused_ok_ = nb_ <= kOctoHeadMaxBlocks && 4 * H <= 1024 && FLAT <= 1024 && H <= 1024 &&
                octo_head_lds_bytes(H, TD, emb_, FLAT) <= 64 * 1024;
    for (int i = 0; i < nb_ && fused_ok_; i++) {
        fused_.d0[i] = hl(blocks_[i].d0);
        fused_.d1[i] = hl(blocks_[i].d1);
        fused_.ln_s[i] = blocks_[i].ln_s;
        fused_.ln_b[i] = blocks_[i].ln_b;
    }
    fused_.ln_eps = 1e-6f;
    fused_.nb = nb_;
    fused_.H = H;
    fused_.TD = TD;
    fused_.emb = emb_;
    fused_.flat = FLAT;
    fused_.steps = steps_;
    fused_.cond = cond_;
    fused_.max_action = max_action_;
    std::vector<float> coef(3 * (size_t)steps_);
    for (int t = 0; t < steps_; t++) {
        coef[3 * t] = a1_[t];
        coef[3 * t + 1] = a2_[t];
        coef[3 * t + 2] = sb_[t];
    }
    fused_.coef = A_.upload(coef.data(), coef.size());
    VLA_HIP_CHECK(hipStreamSynchronize(st));
}

// DiffusionHead::denoise + DiffusionMlp::forward (diffusion_head.cpp:151-177,
// diffusion.cpp:15-36); actions is the running x
void OctoHead::denoise_dev(const float* emb, const float* noise, const float* z, float* actions, hipStream_t st) {
    const char* fe = std::getenv("VLA_OCTO_HEAD_FUSED");  // 0: the layer-by-layer kernels (A/B runs)
    if (fused_ok_ && !(fe && fe[0] == '0' && fe[1] == '\0')) {
        OctoHeadArgs a = fused_;
        a.embv = emb;
        a.noise = noise;
        a.z = z;
        a.actions = actions;
        launch_octo_head(a, st);
        return;
    }
    const int TD = td_, H = H_, FLAT = flat(), IN = TD + emb_ + FLAT;
    Ctx c = ctx_;
    c.st = st;
    copy_f32(actions, noise, FLAT, st);
    for (int s = 0; s < steps_; s++) {
        const int t = steps_ - 1 - s;
        launch_concat3(in_, cond_ + (size_t)t * TD, TD, emb, emb_, actions, FLAT, st);
        linear(c, in_proj_, h_, H, in_, IN, 1);
        for (const Block& B : blocks_) {
            launch_layernorm(n_, h_, B.ln_s, B.ln_b, 1, H, 1e-6f, st);
            linear(c, B.d0, wide_, 4 * H, n_, H, 1, 4);      // silu
            linear(c, B.d1, h_, H, wide_, 4 * H, 1, 0, 1);  // h += ...
        }
        launch_act(h_, H, 4, st);
        linear(c, out_proj_, e_, FLAT, h_, H, 1);
        launch_ddpm_step(actions, e_, z + (size_t)s * FLAT, FLAT, a1_[t], a2_[t], sb_[t], max_action_, st);
    }
}

// ------------------------------------------------------------ the model --

OctoModel::OctoModel(const std::string& dir, const std::string& tok_dir) {
    const CkptFiles files(dir);
    // the tokenizer (t5_tokenizer.cpp:46-72): vocab.txt in tok_dir, through the
    // model's files when tok_dir lies under the model path
    {
        std::string key = dir;
        while (key.size() > 1 && key.back() == '/') key.pop_back();
        const std::string path = tok_dir + "/vocab.txt";
        std::string text;
        if (path.size() > key.size() + 1 && path.compare(0, key.size(), key) == 0 && path[key.size()] == '/') {
            const std::vector<char> b = files.bytes(path.substr(key.size() + 1));
            text.assign(b.begin(), b.end());
        } else {
            const CkptFiles tf(tok_dir);
            const std::vector<char> b = tf.bytes("vocab.txt");
            text.assign(b.begin(), b.end());
        }
        VLA_REQUIRE(tok_.load(text), "octo: vocab.txt in " + tok_dir + " has no pieces");
    }
    const int mask = env_int("OCTO_INT8", 0);  // octo_model.cpp:97
    t5_ = std::make_unique<T5Enc>(files, "t5");
    sp_ = std::make_unique<OctoStem>(files, "stem_primary", mask, 256, 256);
    sw_ = std::make_unique<OctoStem>(files, "stem_wrist", mask, 128, 128);
    tf_ = std::make_unique<OctoTf>(dir, mask & 15);
    head_ = std::make_unique<OctoHead>(files, mask);
    // octo_model.cpp:81-86: the modules must agree
    VLA_REQUIRE(t5_->d_model() == tf_->t5_dim() && head_->emb() == tf_->d() && sp_->embed_dim() == tf_->stem_dim() &&
                    sw_->embed_dim() == tf_->stem_dim() && sp_->tokens() == tf_->tok_primary() &&
                    sw_->tokens() == tf_->tok_wrist(),
                "octo: the T5, stems, transformer and head do not fit together");
    // stats (:88-95): action_dim floats each, finite, std >= 0, mask 0 or 1;
    // a masked-off dimension is left as is (std 1, mean 0 here)
    const int AD = head_->action_dim();
    auto floats = [&](const char* rel) {
        const std::vector<char> b = files.bytes(rel);
        VLA_REQUIRE(b.size() == (size_t)AD * 4, std::string(rel) + ": size does not match action_dim");
        std::vector<float> v(AD);
        std::memcpy(v.data(), b.data(), b.size());
        for (float x : v) VLA_REQUIRE(std::isfinite(x), std::string(rel) + ": non-finite value");
        return v;
    };
    std::vector<float> mean = floats("stats_action_mean.bin"), sd = floats("stats_action_std.bin"),
                       am = floats("stats_action_mask.bin");
    for (int i = 0; i < AD; i++) {
        VLA_REQUIRE(sd[i] >= 0 && (am[i] == 0 || am[i] == 1), "octo: invalid action statistics");
        if (!(am[i] > 0.0f)) {
            sd[i] = 1.0f;
            mean[i] = 0.0f;
        }
    }
    act_mean_ = A_.upload(mean.data(), AD);
    act_std_ = A_.upload(sd.data(), AD);

    const int maxw = tf_->max_horizon(), S = tf_->stem_dim();
    frames_p_ = A_.alloc<uint8_t>((size_t)maxw * 256 * 256 * 3);
    frames_w_ = A_.alloc<uint8_t>((size_t)maxw * 128 * 128 * 3);
    for (int i = 0; i < 2; i++) {
        tok_p_[i] = A_.alloc<float>((size_t)maxw * sp_->tokens() * S);
        tok_w_[i] = A_.alloc<float>((size_t)maxw * sw_->tokens() * S);
    }
    const int FLAT = head_->flat();
    emb_ = A_.alloc<float>(tf_->d());
    noise_ = A_.alloc<float>(FLAT);
    z_ = A_.alloc<float>((size_t)head_->steps() * FLAT);
    act_ = A_.alloc<float>(FLAT);
    out_ = A_.alloc<float>(FLAT);
    VLA_HIP_CHECK(hipStreamCreateWithFlags(&own_, hipStreamNonBlocking));
}

OctoModel::~OctoModel() {
    if (own_) (void)hipStreamDestroy(own_);
}

// OctoModel::lang_encode (octo_model.cpp:143-158): tokenized to n_task ids,
// mask = id != <pad>, encoded once per instruction (at most 64 kept)
const float* OctoModel::lang_dev(const std::string& instruction) {
    const auto it = lang_.find(instruction);
    if (it != lang_.end()) return it->second;
    const int NT = tf_->n_task();
    const std::vector<int32_t> ids = tok_.encode(instruction, NT);
    std::vector<int32_t> am(NT);
    for (int i = 0; i < NT; i++) am[i] = ids[i] != UnigramTokenizer::kPad;
    if (lang_.size() >= 64) {
        VLA_HIP_CHECK(hipStreamSynchronize(own_));
        lang_.clear();
        lang_arena_.clear();
    }
    auto arena = std::make_unique<DeviceArena>();
    float* out = arena->alloc<float>((size_t)NT * t5_->d_model());
    t5_->encode_dev(ids.data(), am.data(), NT, out, own_);
    lang_arena_[instruction] = std::move(arena);
    lang_[instruction] = out;
    return out;
}

void OctoModel::lang(const std::string& instruction, float* out) {
    const float* d = lang_dev(instruction);
    VLA_HIP_CHECK(hipMemcpyAsync(out, d, (size_t)tf_->n_task() * t5_->d_model() * 4, hipMemcpyDeviceToHost, own_));
    VLA_HIP_CHECK(hipStreamSynchronize(own_));
}

// OctoModel::predict (octo_model.cpp:160-229) behind vla_octo_predict_ex's
// checks (octo_capi.cpp:38-58)
void OctoModel::predict(const uint8_t* primary, const uint8_t* wrist, int wnd, const uint8_t* tmask,
                        const std::string& instruction, const float* noise, const float* z, uint64_t seed,
                        bool unnormalize, float* actions) {
    VLA_REQUIRE(primary && tmask && actions, "octo: null buffer");
    if (wnd < 1 || wnd > tf_->max_horizon()) throw ShapeError("octo: wnd must be in [1, max_window]");
    VLA_REQUIRE((noise == nullptr) == (z == nullptr), "octo: pass both noise and z, or neither");
    hipStream_t st = own_;
    const size_t PB = (size_t)256 * 256 * 3, WB = (size_t)128 * 128 * 3;
    const int S = tf_->stem_dim();
    const size_t SP = (size_t)sp_->tokens() * S, SW = (size_t)sw_->tokens() * S;
    // stems: a frame equal to an earlier one of this window, or to one of the
    // previous window, takes its tokens (the values are the same either way)
    const int nxt = cur_ ^ 1;
    auto stems = [&](OctoStem& stem, const uint8_t* img, size_t nb, size_t ns, uint8_t* dev_frames, float* const* toks,
                     const std::vector<uint8_t>& prev) {
        for (int t = 0; t < wnd; t++) {
            const uint8_t* f = img + (size_t)t * nb;
            const float* hit = nullptr;
            for (int u = 0; u < t && !hit; u++)
                if (!std::memcmp(f, img + (size_t)u * nb, nb)) hit = toks[nxt] + (size_t)u * ns;
            for (size_t u = 0; u < prev.size() / nb && !hit; u++)
                if (!std::memcmp(f, prev.data() + u * nb, nb)) hit = toks[cur_] + u * ns;
            float* dst = toks[nxt] + (size_t)t * ns;
            if (hit) {
                copy_f32(dst, hit, (int64_t)ns, st);
            } else {
                VLA_HIP_CHECK(hipMemcpyAsync(dev_frames + (size_t)t * nb, f, nb, hipMemcpyHostToDevice, st));
                stem.encode_dev(dev_frames + (size_t)t * nb, dst, st);
            }
        }
    };
    stems(*sp_, primary, PB, SP, frames_p_, tok_p_, prev_p_);
    if (wrist) stems(*sw_, wrist, WB, SW, frames_w_, tok_w_, prev_w_);
    prev_p_.assign(primary, primary + (size_t)wnd * PB);
    if (wrist) prev_w_.assign(wrist, wrist + (size_t)wnd * WB);
    else prev_w_.clear();
    cur_ = nxt;

    const float* t5 = lang_dev(instruction);
    tf_->forward_dev(t5, tok_p_[cur_], wrist ? tok_w_[cur_] : nullptr, wnd, tmask, emb_, st);

    // DDPM noise: N(0, 1) floats from mt19937_64(seed), the initial x then
    // steps x flat per-step draws (:207-219)
    const int FLAT = head_->flat(), steps = head_->steps();
    std::vector<float> nbuf, zbuf;
    if (!noise) {
        std::mt19937_64 rng(seed);
        std::normal_distribution<float> nd(0.0f, 1.0f);
        nbuf.resize(FLAT);
        zbuf.resize((size_t)steps * FLAT);
        for (float& v : nbuf) v = nd(rng);
        for (float& v : zbuf) v = nd(rng);
        noise = nbuf.data();
        z = zbuf.data();
    }
    VLA_HIP_CHECK(hipMemcpyAsync(noise_, noise, (size_t)FLAT * 4, hipMemcpyHostToDevice, st));
    VLA_HIP_CHECK(hipMemcpyAsync(z_, z, (size_t)steps * FLAT * 4, hipMemcpyHostToDevice, st));
    head_->denoise_dev(emb_, noise_, z_, act_, st);
    const float* res = act_;
    if (unnormalize) {  // v * std + mean where the mask is set (:221-228)
        launch_unnormalize(out_, act_, head_->action_dim(), head_->horizon(), head_->action_dim(), act_mean_, act_std_,
                           0.0f, st);
        res = out_;
    }
    VLA_HIP_CHECK(hipMemcpyAsync(actions, res, (size_t)FLAT * 4, hipMemcpyDeviceToHost, st));
    VLA_HIP_CHECK(hipStreamSynchronize(st));
}

}  // namespace hip
}  // namespace vla
