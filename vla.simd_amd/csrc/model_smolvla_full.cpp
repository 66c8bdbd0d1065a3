// model_smolvla_full.cpp - SmolVLA end to end on the device (see models.h).
//
// Follows src/models/smolvla/smolvla_model.cpp (heads.meta, emb.bin,
// heads.bin, the stats files; the prefix assembly and the state/action
// normalization of predict_normalized / predict) and smolvla_capi.cpp (the
// tokenizer call, config.txt, resize_with_pad, the default noise, the
// argument checks). The vision tower, the prefix tower and the denoise loop
// are SiglipTf and SmolvlaTf; the image, embedding and normalization steps
// are the kernels of policy.hip, all on one stream.
#include "ckpt.h"
#include "models.h"

#include <cmath>
#include <cstdlib>
#include <fstream>
#include <random>
#include <sstream>

namespace vla {
namespace hip {

namespace {

bool shape_fits2(int a, int b) { return a > 0 && b > 0 && (int64_t)a * b <= 2147483647LL; }

// arena.h metadata_int: a finite whole number within int
int meta_whole(const std::string& key, double v) {
    VLA_REQUIRE(std::isfinite(v) && v == std::trunc(v) && v >= -2147483648.0 && v <= 2147483647.0,
                "heads.meta: " + key + " is not an integer");
    return (int)v;
}

// int_env as hal::env::int_env reads SMOLVLA_INT8 (env.cpp:23-29)
int env_int(const char* name, int dflt) {
    const char* e = std::getenv(name);
    if (!e || !*e) return dflt;
    char* end = nullptr;
    const long long v = std::strtoll(e, &end, 10);
    return *end || v < -2147483648LL || v > 2147483647LL ? dflt : (int)v;
}

std::string strip_slash(std::string p) {
    while (p.size() > 1 && p.back() == '/') p.pop_back();
    return p;
}

// A file of the tokenizer directory: through the model's files (GGUF entry or
// sidecar) when tok_dir lies under the model path, as the reference's mount
// resolves it (files.cpp:147-166), else from disk.
std::string tok_file(const CkptFiles& model, const std::string& model_dir, const std::string& tok_dir,
                     const char* name) {
    const std::string key = strip_slash(model_dir), path = tok_dir + "/" + name;
    if (path.size() > key.size() + 1 && path.compare(0, key.size(), key) == 0 && path[key.size()] == '/') {
        const std::string rel = path.substr(key.size() + 1);
        if (model.size(rel) < 0) throw ArgError("smolvla: cannot load the tokenizer from " + tok_dir);
        const std::vector<char> b = model.bytes(rel);
        return std::string(b.begin(), b.end());
    }
    std::ifstream f(path, std::ios::binary);
    if (!f) throw ArgError("smolvla: cannot load the tokenizer from " + tok_dir + " (vocab.txt, merges.txt)");
    std::ostringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

std::vector<float> floats_of(const CkptFiles& files, const std::string& rel, size_t n) {
    const std::vector<char> b = files.bytes(rel);
    VLA_REQUIRE(b.size() == n * 4, rel + ": size does not match heads.meta");
    std::vector<float> v(n);
    std::memcpy(v.data(), b.data(), b.size());
    for (float x : v) VLA_REQUIRE(std::isfinite(x), rel + ": non-finite value");
    return v;
}

}  // namespace

SmolvlaModel::SmolvlaModel(const std::string& dir, const std::string& tok_dir) {
    const CkptFiles files(dir);
    const int mask = env_int("SMOLVLA_INT8", 0);  // smolvla_model.cpp:111
    vit_ = std::make_unique<SiglipTf>(dir, mask & 15);
    tf_ = std::make_unique<SmolvlaTf>(dir, mask & 48);

    // heads.meta (smolvla_model.cpp:56-85): "key value" pairs, every value a
    // finite number, the integer keys whole numbers
    int max_state_dim = 32, n_views = 2;
    double eps = 1e-8;
    {
        const std::vector<char> b = files.bytes("heads.meta");
        std::istringstream in(std::string(b.begin(), b.end()));
        std::string k;
        double v;
        while (in >> k) {
            VLA_REQUIRE(static_cast<bool>(in >> v) && std::isfinite(v), "heads.meta: bad value for key " + k);
            if (k == "vocab") vocab_ = meta_whole(k, v);
            else if (k == "hidden") hidden_ = meta_whole(k, v);
            else if (k == "max_state_dim") max_state_dim = meta_whole(k, v);
            else if (k == "real_state_dim") real_state_dim_ = meta_whole(k, v);
            else if (k == "real_action_dim") real_action_dim_ = meta_whole(k, v);
            else if (k == "n_views") n_views = meta_whole(k, v);
            else if (k == "norm_eps") eps = v;
        }
    }
    max_state_dim_ = max_state_dim;
    n_views_ = n_views;
    norm_eps_ = (float)eps;
    VLA_REQUIRE(shape_fits2(vocab_, hidden_) && shape_fits2(max_state_dim_, hidden_) && n_views_ > 0 &&
                    std::isfinite(norm_eps_) && norm_eps_ > 0 && real_state_dim_ > 0 &&
                    real_state_dim_ <= max_state_dim_ && real_action_dim_ > 0 &&
                    real_action_dim_ <= tf_->max_action_dim() && hidden_ == tf_->hidden() &&
                    hidden_ == vit_->out_dim(),
                "heads.meta is missing or malformed (smolvla_model.cpp:67-81 bounds)");
    VLA_REQUIRE(hidden_ % 4 == 0, "heads.meta: the device path needs hidden a multiple of 4");

    // emb.bin (bf16 [vocab, hidden]) and heads.bin (state_proj [hidden,
    // max_state_dim] + bias [hidden]), sizes exact (:83-99)
    {
        const std::vector<char> b = files.bytes("emb.bin");
        VLA_REQUIRE(b.size() == (size_t)vocab_ * hidden_ * 2, "emb.bin: size does not match heads.meta");
        emb_ = A_.upload(reinterpret_cast<const uint16_t*>(b.data()), (size_t)vocab_ * hidden_);
    }
    {
        const std::vector<char> b = files.bytes("heads.bin");
        const size_t nw = (size_t)hidden_ * max_state_dim_;
        VLA_REQUIRE(b.size() == (nw + hidden_) * 4, "heads.bin: size does not match heads.meta");
        const float* p = reinterpret_cast<const float*>(b.data());
        state_w_ = A_.upload(p, nw);
        state_b_ = A_.upload(p + nw, hidden_);
    }
    // the statistics (:101-112): exact sizes, finite, standard deviations >= 0
    const std::vector<float> sm = floats_of(files, "stats_state_mean.bin", real_state_dim_);
    const std::vector<float> ss = floats_of(files, "stats_state_std.bin", real_state_dim_);
    const std::vector<float> am = floats_of(files, "stats_action_mean.bin", real_action_dim_);
    const std::vector<float> as = floats_of(files, "stats_action_std.bin", real_action_dim_);
    for (const auto* v : {&ss, &as})
        for (float x : *v) VLA_REQUIRE(x >= 0, "smolvla: negative standard deviation in the stats");
    state_mean_ = A_.upload(sm.data(), sm.size());
    state_std_ = A_.upload(ss.data(), ss.size());
    action_mean_ = A_.upload(am.data(), am.size());
    action_std_ = A_.upload(as.data(), as.size());

    // the tokenizer (smolvla_capi.cpp:80-84) and config.txt's optional keys
    // (:43-66): one line per key, split at the first space, a value std::stoi
    // cannot read keeps the default
    tok_ = std::make_unique<BpeTokenizer>();
    VLA_REQUIRE(tok_->load(tok_file(files, dir, tok_dir, "vocab.txt"), tok_file(files, dir, tok_dir, "merges.txt")),
                "smolvla: cannot load the tokenizer from " + tok_dir + " (vocab.txt, merges.txt)");
    if (files.size("config.txt") >= 0) {
        const std::vector<char> b = files.bytes("config.txt");
        std::istringstream in(std::string(b.begin(), b.end()));
        std::string line;
        while (std::getline(in, line)) {
            if (!line.empty() && line.back() == '\r') line.pop_back();
            const size_t sp = line.find(' ');
            if (sp == std::string::npos) continue;
            const std::string k = line.substr(0, sp), v = line.substr(sp + 1);
            try {
                if (k == "tokenizer_max_length") tok_maxlen_ = std::stoi(v);
                else if (k == "pad_token_id") pad_id_ = std::stoi(v);
            } catch (const std::exception&) {
            }
        }
        if (tok_maxlen_ < 1) tok_maxlen_ = 48;
    }

    // fixed-size buffers
    const int S = vit_->img(), C = tf_->chunk(), MAD = tf_->max_action_dim();
    pixels_ = A_.alloc<float>((size_t)n_views_ * 3 * S * S);
    state_raw_ = A_.alloc<float>(real_state_dim_);
    state_n_ = A_.alloc<float>(max_state_dim_);  // zero past real_state_dim, never written there
    noise_ = A_.alloc<float>((size_t)C * MAD);
    act_n_ = A_.alloc<float>((size_t)C * MAD);
    actions_ = A_.alloc<float>((size_t)C * real_action_dim_);
    guide_ = A_.alloc<float>((size_t)C * MAD);  // zero past real_action_dim, never written there
    prev_ = A_.alloc<float>((size_t)C * real_action_dim_);
    weights_ = A_.alloc<float>(C);
    VLA_HIP_CHECK(hipStreamCreateWithFlags(&own_, hipStreamNonBlocking));
}

SmolvlaModel::~SmolvlaModel() {
    if (own_) (void)hipStreamDestroy(own_);
}

// vla_smolvla_tokenize (smolvla_capi.cpp:100-121): at most the last 64 KiB of
// the text, trailing newlines replaced by exactly one, the last tok_maxlen ids
int SmolvlaModel::tokenize(const std::string& text, int32_t* ids, int32_t* mask) const {
    std::string s = text.size() > 65536 ? text.substr(text.size() - 65536) : text;
    while (!s.empty() && s.back() == '\n') s.pop_back();
    s.push_back('\n');
    std::vector<int32_t> enc = tok_->encode(s);
    if ((int)enc.size() > tok_maxlen_) enc.erase(enc.begin(), enc.end() - tok_maxlen_);
    for (int i = 0; i < tok_maxlen_; i++) {
        ids[i] = i < (int)enc.size() ? enc[i] : pad_id_;
        mask[i] = i < (int)enc.size() ? 1 : 0;
    }
    return (int)enc.size();
}

void SmolvlaModel::stage_frames(const uint8_t* frames, int nv, int height, int width) {
    const size_t bytes = (size_t)nv * height * width * 3;
    if (bytes > frames_cap_) {
        VLA_HIP_CHECK(hipStreamSynchronize(own_));
        F_ = std::make_unique<DeviceArena>();
        frames_ = F_->alloc<uint8_t>(bytes);
        frames_cap_ = bytes;
    }
    VLA_HIP_CHECK(hipMemcpyAsync(frames_, frames, bytes, hipMemcpyHostToDevice, own_));
    launch_resize_with_pad(pixels_, frames_, nv, height, width, vit_->img(), own_);
}

void SmolvlaModel::preprocess(const uint8_t* frames, int nv, int height, int width, float* pixels) {
    VLA_REQUIRE(frames && pixels && height > 0 && width > 0, "smolvla: bad frames");
    VLA_REQUIRE(nv == n_views_, "smolvla: n_views differs from the checkpoint's");
    stage_frames(frames, nv, height, width);
    const size_t n = (size_t)nv * 3 * vit_->img() * vit_->img();
    VLA_HIP_CHECK(hipMemcpyAsync(pixels, pixels_, n * 4, hipMemcpyDeviceToHost, own_));
    VLA_HIP_CHECK(hipStreamSynchronize(own_));
}

// smolvla_capi.cpp:123-167 + SmolvlaModel::predict / predict_normalized
// (smolvla_model.cpp:183-291)
void SmolvlaModel::predict(const uint8_t* frames, int nv, int height, int width, const int32_t* tokens,
                           const int32_t* lang_mask, int n_lang, const float* state, const float* noise,
                           uint64_t seed, float* actions, const float* prev, int n_prev, const float* weights,
                           float max_guidance) {
    VLA_REQUIRE(frames && tokens && lang_mask && state && actions, "smolvla: null buffer");
    VLA_REQUIRE(height > 0 && width > 0 && n_lang >= 0 && n_prev >= 0, "smolvla: bad frame size or counts");
    if (!prev) n_prev = 0;
    VLA_REQUIRE(n_prev == 0 || (weights && std::isfinite(max_guidance) && max_guidance > 0),
                "smolvla: guidance needs weights and a positive finite max_guidance");
    const int C = tf_->chunk(), MAD = tf_->max_action_dim(), ad = real_action_dim_, H = hidden_;
    if (nv != n_views_ || n_prev > C) throw ShapeError("smolvla: n_views or n_prev does not fit the checkpoint");
    for (int i = 0; n_prev > 0 && i < C; i++) VLA_REQUIRE(std::isfinite(weights[i]), "smolvla: non-finite weight");
    for (size_t i = 0; i < (size_t)n_prev * ad; i++)
        VLA_REQUIRE(std::isfinite(prev[i]), "smolvla: non-finite previous action");
    for (int t = 0; t < n_lang; t++)
        if (tokens[t] < 0 || tokens[t] >= vocab_)
            throw ShapeError("smolvla: token id " + std::to_string(tokens[t]) + " is outside the vocabulary");
    // pad: images and state real, the language tokens their mask
    // (smolvla_model.cpp:246-249); the device graph takes 0/1 only
    const int TOK = vit_->n_tokens(), n_img = nv * TOK, np = n_img + n_lang + 1;
    std::vector<int32_t> pad(np, 1);
    for (int t = 0; t < n_lang; t++) pad[n_img + t] = lang_mask[t];

    // the default noise: N(0, 1) floats from mt19937_64(seed) (:140-147)
    std::vector<float> nbuf;
    if (!noise) {
        nbuf.resize((size_t)C * MAD);
        std::mt19937_64 rng(seed);
        std::normal_distribution<float> nd(0.0f, 1.0f);
        for (float& x : nbuf) x = nd(rng);
        noise = nbuf.data();
    }

    hipStream_t st = own_;
    if (np > prefix_cap_) {
        VLA_HIP_CHECK(hipStreamSynchronize(st));
        P_ = std::make_unique<DeviceArena>();
        prefix_ = P_->alloc<float>((size_t)np * H);
        ids_ = P_->alloc<int32_t>(n_lang > 0 ? n_lang : 1);
        prefix_cap_ = np;
    }
    stage_frames(frames, nv, height, width);
    // prefix rows: the views' image tokens x sqrt(H), the language embeddings
    // x sqrt(H), the projected state (:218-240)
    const float sq = std::sqrt((float)H);
    const size_t per_view = (size_t)3 * vit_->img() * vit_->img();
    for (int v = 0; v < nv; v++) vit_->encode_dev(pixels_ + v * per_view, prefix_ + (size_t)v * TOK * H, st);
    launch_scale(prefix_, (int64_t)n_img * H, sq, st);
    if (n_lang > 0) {
        VLA_HIP_CHECK(hipMemcpyAsync(ids_, tokens, (size_t)n_lang * 4, hipMemcpyHostToDevice, st));
        launch_embed_bf16(prefix_ + (size_t)n_img * H, emb_, ids_, n_lang, H, sq, st);
    }
    VLA_HIP_CHECK(hipMemcpyAsync(state_raw_, state, (size_t)real_state_dim_ * 4, hipMemcpyHostToDevice, st));
    launch_normalize_pad(state_n_, max_state_dim_, state_raw_, 1, 1, real_state_dim_, state_mean_, state_std_,
                         norm_eps_, st);
    launch_linear_f32(prefix_ + (size_t)(np - 1) * H, H, state_n_, max_state_dim_, state_w_, max_state_dim_, state_b_,
                      1, H, max_state_dim_, 0, 0, 1.0f, st);
    VLA_HIP_CHECK(hipMemcpyAsync(noise_, noise, (size_t)C * MAD * 4, hipMemcpyHostToDevice, st));

    SmolvlaTf::Rtc rtc{guide_, weights_, max_guidance};
    if (n_prev > 0) {  // the normalized previous chunk, zero-padded (:268-276)
        VLA_HIP_CHECK(hipMemcpyAsync(prev_, prev, (size_t)n_prev * ad * 4, hipMemcpyHostToDevice, st));
        VLA_HIP_CHECK(hipMemcpyAsync(weights_, weights, (size_t)C * 4, hipMemcpyHostToDevice, st));
        launch_normalize_pad(guide_, MAD, prev_, n_prev, C, ad, action_mean_, action_std_, norm_eps_, st);
    }
    tf_->chunk_dev(prefix_, pad.data(), np, noise_, act_n_, st, n_prev > 0 ? &rtc : nullptr);
    // un-normalized, the first real_action_dim columns of each row (:280-290)
    launch_unnormalize(actions_, act_n_, MAD, C, ad, action_mean_, action_std_, norm_eps_, st);
    VLA_HIP_CHECK(hipMemcpyAsync(actions, actions_, (size_t)C * ad * 4, hipMemcpyDeviceToHost, st));
    VLA_HIP_CHECK(hipStreamSynchronize(st));
}

}  // namespace hip
}  // namespace vla
