// model_impact.cpp - IMPACT end to end on the device (see models.h).
//
// Follows src/models/impact/impact_model.cpp (load, set_instruction, predict)
// and t5_text.cpp (text.meta, the tail of text.bin, vocab_map.bin, the
// remap, encode). The vision trunk, the transformer, the normalizations and
// the un-normalization are ActModel's with the IMPACT spec; this file adds
// the language pathway, which runs once per instruction: tokenize and remap
// on the host, then T5-small, the text projection, the mask-aware mean pool
// and the FiLM head on the device. Its outputs stay on the device: the text
// tokens feed the transformer's text tail and gamma / beta land in the
// trunk's FiLM buffers.
#include "ckpt.h"
#include "models.h"

#include <climits>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <sstream>

namespace vla {
namespace hip {

namespace {

// arena.h metadata_int: a finite whole number within int, else an error
int meta_int(const std::string& file, const std::string& key, double v) {
    VLA_REQUIRE(std::isfinite(v) && v == std::trunc(v) && v >= (double)INT_MIN && v <= (double)INT_MAX,
                file + ": " + key + " is not an integer");
    return (int)v;
}

bool dims_fit(std::initializer_list<int> dims) {
    int count = 1;
    for (int d : dims) {
        if (d <= 0 || count > INT_MAX / d) return false;
        count *= d;
    }
    return true;
}

// The values after a key, read as the reference's loaders read them: each
// `ss >> v` must succeed and nothing but whitespace may follow the last one.
template <class T>
void read_one(const std::string& file, const std::string& key, const std::string& text, T& v) {
    std::istringstream ss(text);
    ss >> v;
    VLA_REQUIRE(!ss.fail() && (ss >> std::ws).eof(), file + ": bad value for key " + key + ": '" + text + "'");
}

}  // namespace

ImpactModel::ImpactModel(const std::string& dir) {
    const CkptFiles files(dir);

    // config.txt: the keys ActModel does not read (impact_model.cpp:27-46)
    for (const auto& kv : files.meta_lines("config.txt")) {
        if (kv.first == "vocab_full") read_one("config.txt", kv.first, kv.second, vocab_full_);
        else if (kv.first == "unk_id") read_one("config.txt", kv.first, kv.second, unk_id_);
    }

    // the trunk (vision.meta / .bin, FiLM points), the transformer
    // (impact.meta / .bin, int8_state) and stats.bin (:50-66, :98-136)
    ActSpec spec;
    spec.backbone = "vision";
    spec.tf = "impact";
    spec.int8_env = "IMPACT_INT8";
    spec.conv_from_env = "IMPACT_I8_CONV_FROM";
    spec.conv_to_env = "IMPACT_I8_CONV_TO";
    spec.int8_state = true;
    spec.film = true;
    act_ = std::make_unique<ActModel>(dir, spec);

    // the tokenizer (t5_tokenizer.cpp:46-72): vocab.txt in the model directory
    {
        const std::vector<char> b = files.bytes("vocab.txt");
        VLA_REQUIRE(tok_.load(std::string(b.begin(), b.end())), "impact: vocab.txt has no pieces");
    }

    // text.meta / text.bin (t5_text.cpp:19-64): the T5 encoder, then the
    // projection [proj_dim, d_model] + bias, the text positions [n_text,
    // proj_dim] and the FiLM head [2 film_total, d_model] + bias
    std::vector<float> tail;
    t5_ = std::make_unique<T5Enc>(files, "text", &tail);
    int encoder_floats = 0;
    {
        const std::vector<char> b = files.bytes("text.meta");
        std::istringstream in(std::string(b.begin(), b.end()));
        std::string key;
        double val;
        while (in >> key) {
            VLA_REQUIRE(static_cast<bool>(in >> val) && std::isfinite(val), "text.meta: bad value for key " + key);
            if (key == "proj_dim") proj_dim_ = meta_int("text.meta", key, val);
            else if (key == "n_text") n_text_ = meta_int("text.meta", key, val);
            else if (key == "film_total") film_total_ = meta_int("text.meta", key, val);
            else if (key == "encoder_floats") encoder_floats = meta_int("text.meta", key, val);
        }
    }
    const int64_t total = files.size("text.bin") / 4;
    const size_t enc_end = (size_t)total - tail.size();
    VLA_REQUIRE(encoder_floats <= 0 || (size_t)encoder_floats == enc_end,
                "impact: text.bin's encoder length differs from text.meta's encoder_floats");
    const int D = t5_->d_model(), P = proj_dim_, T = n_text_, F = film_total_;
    VLA_REQUIRE(dims_fit({P, T}) && dims_fit({P, D}) && F >= 0 && (F == 0 || dims_fit({2, F, D})),
                "impact: text.meta is missing proj_dim / n_text / film_total");
    const size_t want = ((size_t)P * D + P) + (size_t)T * P + ((size_t)2 * F * D + (size_t)2 * F);
    VLA_REQUIRE(tail.size() == want, "impact: text.bin's heads do not match text.meta");
    const float* p = tail.data();
    proj_w_ = A_.upload(p, (size_t)P * D);
    proj_b_ = A_.upload(p + (size_t)P * D, P);
    p += (size_t)P * D + P;
    text_pos_ = A_.upload(p, (size_t)T * P);
    p += (size_t)T * P;
    if (F) {
        film_w_ = A_.upload(p, (size_t)2 * F * D);
        film_bias_ = A_.upload(p + (size_t)2 * F * D, (size_t)2 * F);
    }

    // vocab_map.bin: one int32 per full-vocabulary id (t5_text.cpp:66-91)
    {
        VLA_REQUIRE(vocab_full_ > 0 && (size_t)vocab_full_ <= SIZE_MAX / 4, "config.txt: invalid vocab_full");
        const std::vector<char> b = files.bytes("vocab_map.bin");
        VLA_REQUIRE(b.size() == (size_t)vocab_full_ * 4, "impact: vocab_map.bin's size differs from vocab_full");
        vocab_map_.resize(vocab_full_);
        std::memcpy(vocab_map_.data(), b.data(), b.size());
        VLA_REQUIRE(unk_id_ >= 0 && unk_id_ < vocab_full_ && vocab_map_[unk_id_] >= 0,
                    "impact: <unk> is not in the pruned vocabulary");
        for (int32_t id : vocab_map_)
            VLA_REQUIRE(id >= -1 && id < t5_->vocab(), "impact: vocab_map.bin names an id outside the table");
        unk_compact_ = vocab_map_[unk_id_];
    }

    // the modules must agree (impact_model.cpp:73-96)
    VLA_REQUIRE(F == act_->film_total(), "impact: the FiLM head and the trunk's film_after points disagree");
    VLA_REQUIRE(T == act_->tf_n_text(), "impact: the text tower's n_text differs from the transformer's");
    VLA_REQUIRE(P == act_->tf_dim(), "impact: the text projection's width differs from the transformer's");

    h_ = A_.alloc<float>((size_t)T * D);
    text_tok_ = A_.alloc<float>((size_t)T * P);
    pooled_ = A_.alloc<float>(D);
    gb_ = A_.alloc<float>(F ? (size_t)2 * F : 1);
    mask_d_ = A_.alloc<int32_t>(T);
    VLA_HIP_CHECK(hipStreamCreateWithFlags(&own_, hipStreamNonBlocking));
}

ImpactModel::~ImpactModel() {
    if (own_) (void)hipStreamDestroy(own_);
}

// ImpactText::remap (t5_text.cpp:94-111): ids outside the pruned table -> <unk>
int ImpactModel::remap(const std::vector<int32_t>& ids, std::vector<int32_t>& compact) {
    int oov = 0;
    compact.resize(ids.size());
    for (size_t t = 0; t < ids.size(); t++) {
        const int32_t id = ids[t];
        const int32_t c = (id >= 0 && id < (int32_t)vocab_map_.size()) ? vocab_map_[id] : -1;
        compact[t] = c < 0 ? unk_compact_ : c;
        oov += c < 0;
    }
    if (oov && !warned_oov_) {
        warned_oov_ = true;
        std::fprintf(stderr,
                     "impact: instruction contains %d token(s) outside the pruned vocabulary; substituting <unk>. "
                     "The language pathway is blind to those words.\n",
                     oov);
    }
    return oov;
}

// ImpactModel::set_instruction (impact_model.cpp:138-170) + ImpactText::encode
// (t5_text.cpp:113-150)
void ImpactModel::set_instruction(const std::string& instruction) {
    if (have_text_ && instruction == cached_) return;
    const int L = n_text_, D = t5_->d_model(), P = proj_dim_, F = film_total_;
    ids_ = tok_.encode(instruction, L);
    ids_.resize(L, UnigramTokenizer::kPad);
    // 1 for each token up to the first <pad>: padded rows are still encoded,
    // the mask decides where the tower may attend
    mask_.assign(L, 0);
    n_real_ = 0;
    for (int i = 0; i < L; i++) {
        if (ids_[i] == UnigramTokenizer::kPad) break;
        mask_[i] = 1;
        n_real_ = i + 1;
    }
    remap(ids_, compact_);

    hipStream_t st = own_;
    t5_->encode_dev(compact_.data(), mask_.data(), L, h_, st);
    // text tokens: the projection only (the positions ride in the transformer's
    // pos array, added to queries and keys)
    launch_linear_f32(text_tok_, P, h_, D, proj_w_, D, proj_b_, L, P, D, 0, 0, 1.0f, st);
    gamma_.assign(F, 0.0f);
    beta_.assign(F, 0.0f);
    if (F) {
        VLA_HIP_CHECK(hipMemcpyAsync(mask_d_, mask_.data(), (size_t)L * 4, hipMemcpyHostToDevice, st));
        launch_masked_row_mean(pooled_, h_, D, mask_d_, L, D, st);
        launch_linear_f32(gb_, 2 * F, pooled_, D, film_w_, D, film_bias_, 1, 2 * F, D, 0, 0, 1.0f, st);
        VLA_HIP_CHECK(hipMemcpyAsync(act_->film_gamma(), gb_, (size_t)F * 4, hipMemcpyDeviceToDevice, st));
        VLA_HIP_CHECK(hipMemcpyAsync(act_->film_beta(), gb_ + F, (size_t)F * 4, hipMemcpyDeviceToDevice, st));
        VLA_HIP_CHECK(hipMemcpyAsync(gamma_.data(), gb_, (size_t)F * 4, hipMemcpyDeviceToHost, st));
        VLA_HIP_CHECK(hipMemcpyAsync(beta_.data(), gb_ + F, (size_t)F * 4, hipMemcpyDeviceToHost, st));
    }
    // the host mask and the host copies must be complete before this returns
    VLA_HIP_CHECK(hipStreamSynchronize(st));
    cached_ = instruction;
    have_text_ = true;
}

// ImpactModel::predict (impact_model.cpp:201-244): device pointers, the
// instruction already set
void ImpactModel::predict_dev(const uint8_t* frames, const float* state, bool unnormalize, float* actions,
                              hipStream_t caller) {
    VLA_REQUIRE(have_text_, "impact: predict before set_instruction (IMPACT is instruction-conditioned)");
    act_->predict_text_dev(frames, state, text_tok_, text_pos_, n_real_, unnormalize, actions, caller);
}

}  // namespace hip
}  // namespace vla
