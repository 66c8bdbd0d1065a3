/*
 * ref_models_shim.cpp - extern "C" wrapper over the REAL reference policy
 * graphs (ActTransformer, OctoTransformer, SmollmVlm + ActionExpert), compiled
 * from the reference's own sources where they lie (oracle/Makefile names them)
 * into oracle/_ref/libvla_ref.so next to ref_shim.cpp.
 *
 * TEST INFRASTRUCTURE ONLY: the graph parity tests load the same checkpoint
 * files into these and into the device graphs and compare the outputs. The
 * product never loads it.
 *
 * Beyond forwarding, this file does what the reference's model classes do
 * around the graphs and that the tests need without images or tokenizers:
 *   - the io::Mount of the model path (act_model.cpp:23, octo_model.cpp:66,
 *     smolvla_model.cpp:54), so a vla.simd GGUF loads through the reference's
 *     own reader; ref_mount_read exposes that reader's bytes for one file;
 *   - the OCTO_INT8 / SMOLVLA_INT8 per-layer init_int8 calls of
 *     OctoModel::apply_int8 (src/models/octo/octo_model.cpp:104-140) and
 *     SmolvlaModel::apply_int8 (src/models/smolvla/smolvla_model.cpp:111-155),
 *     with the mask passed in instead of read from the environment;
 *   - the prefix-LM mask, positions and denoise mask of
 *     SmolvlaModel::predict_normalized (smolvla_model.cpp:252-275) built from a
 *     pad vector, so the chunk starts from given prefix embeddings;
 *   - the whole SmolvlaModel with SMOLVLA_INT8's groups for a given mask and
 *     the body of vla_smolvla_predict_rtc (smolvla_capi.cpp:123-167) around
 *     it, since SmolvlaModel::apply_int8 latches the variable once per
 *     process (a static); the library's own vla_smolvla_* entry points
 *     (compiled in from smolvla_capi.cpp) serve the environment's mask;
 *   - resize_with_pad and the BPE tokenizer on their own;
 *   - the whole OctoModel with OCTO_INT8's groups for a given mask
 *     (OctoModel::apply_int8, octo_model.cpp:100-141, latches the variable
 *     once per process too) and OctoModel::predict restated over its public
 *     parts (octo_model.cpp:160-229, without the frame reuse, which changes
 *     no value), with an optional 1-ulp perturbation of the stem tokens.
 */
#include "io/files.h"
#include "models/act/act_model.h"
#include "models/act/act_transformer.h"
#include "models/octo/octo_model.h"
#include "models/octo/octo_transformer.h"
#include "models/smolvla/action_expert.h"
#include "models/smolvla/siglip_vision.h"
#include "models/smolvla/smollm2_lm.h"
#include "models/smolvla/smolvla_model.h"
#include "ops/lm_ops.h"
#include "preprocess/image.h"
#include "tokenizer/t5_tokenizer.h"
#include "tokenizer/tokenizer.h"

#include <cmath>
#include <cstdint>
#include <cstring>
#include <iterator>
#include <string>
#include <cstdio>
#include <exception>
#include <limits>
#include <vector>

#define REF_API extern "C" __attribute__((visibility("default")))

using namespace tcpu;

REF_API void* ref_act_load(const char* dir, int img_ch, int int8_mask) {
    try {
        const io::Mount mount(dir);
        if (!mount.ok()) return nullptr;
        auto* t = new ActTransformer();
        if (!t->load(dir, img_ch, int8_mask)) {
            delete t;
            return nullptr;
        }
        return t;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_act_load: %s\n", e.what());
        return nullptr;
    }
}

/* The bytes of <path>/<rel> as the reference's loaders see them (a mounted
 * GGUF's generated file, else the file on disk): the size, or -1 when there
 * is no such file, -2 when the path does not mount; copies min(size, cap). */
REF_API long long ref_mount_read(const char* path, const char* rel, char* buf, long long cap) {
    try {
        const io::Mount mount(path);
        if (!mount.ok()) return -2;
        io::InFile f(std::string(path) + "/" + rel, std::ios::binary);
        if (!f) return -1;
        std::string all((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
        const long long n = (long long)all.size();
        if (buf && cap > 0) std::memcpy(buf, all.data(), (size_t)(n < cap ? n : cap));
        return n;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_mount_read: %s\n", e.what());
        return -2;
    }
}

REF_API void ref_act_free(void* h) { delete static_cast<ActTransformer*>(h); }

/* IMPACT's transformer: load with int8_state (impact_model.cpp:65) and run
 * with a text tail (act_transformer.cpp:343-360). */
REF_API void* ref_act_load_ex(const char* dir, int img_ch, int int8_mask, int int8_state) {
    try {
        const io::Mount mount(dir);
        if (!mount.ok()) return nullptr;
        auto* t = new ActTransformer();
        if (!t->load(dir, img_ch, int8_mask, int8_state != 0)) {
            delete t;
            return nullptr;
        }
        return t;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_act_load_ex: %s\n", e.what());
        return nullptr;
    }
}

REF_API int ref_act_forward_text(void* h, const float* feats, int n_cams, int fh, int fw, const float* state_norm,
                                 const float* text, const float* text_pos, int n_text_real, float* actions_norm) {
    auto* t = static_cast<ActTransformer*>(h);
    const int img_ch = t->img_proj.K;
    std::vector<const float*> cams(n_cams);
    for (int c = 0; c < n_cams; c++) cams[c] = feats + (size_t)c * fh * fw * img_ch;
    t->forward(cams.data(), n_cams, fh, fw, state_norm, actions_norm, text, text_pos, n_text_real);
    return 0;
}

REF_API int ref_act_forward(void* h, const float* feats, int n_cams, int fh, int fw,
                            const float* state_norm, float* actions_norm) {
    auto* t = static_cast<ActTransformer*>(h);
    const int img_ch = t->img_proj.K;
    std::vector<const float*> cams(n_cams);
    for (int c = 0; c < n_cams; c++) cams[c] = feats + (size_t)c * fh * fw * img_ch;
    t->forward(cams.data(), n_cams, fh, fw, state_norm, actions_norm);
    return 0;
}

REF_API void* ref_octo_load(const char* dir, int int8_mask) {
    try {
        const io::Mount mount(dir);
        if (!mount.ok()) return nullptr;
        auto* t = new OctoTransformer();
        if (!t->load(dir)) {
            delete t;
            return nullptr;
        }
        for (nn::EncoderLayer& l : t->layers) {
            if (int8_mask & 1) {
                l.attn.wq.init_int8();
                l.attn.wk.init_int8();
                l.attn.wv.init_int8();
                l.attn.wo.init_int8();
            }
            if (int8_mask & 2) l.w1.init_int8();
            if (int8_mask & 4) l.w2.init_int8();
        }
        if (int8_mask & 8) {
            t->proj_task.init_int8();
            t->proj_prim.init_int8();
            t->proj_wrist.init_int8();
        }
        return t;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_octo_load: %s\n", e.what());
        return nullptr;
    }
}

REF_API void ref_octo_free(void* h) { delete static_cast<OctoTransformer*>(h); }

/* out [total_tokens(wnd), d]; only the readout row is written */
REF_API int ref_octo_forward(void* h, const float* t5, const float* stem_p, const float* stem_w, int wnd,
                             const uint8_t* tmask, float* out) {
    auto* t = static_cast<OctoTransformer*>(h);
    t->forward(t5, stem_p, stem_w, wnd, tmask, out);
    return t->readout_index(wnd, wnd - 1);
}

REF_API int ref_octo_total_tokens(void* h, int wnd) {
    return static_cast<OctoTransformer*>(h)->total_tokens(wnd);
}

/* OctoTransformer::forward (octo_transformer.cpp:144-219) driven over either
 * token layout: repeat_task 1 is the reference's own (each timestep repeats
 * the task tokens, 690 tokens at the Octo-base config; the result must equal
 * ref_octo_forward bit for bit), repeat_task 0 drops the per-step copy (the
 * 658-token layout), which the reference's forward cannot produce. The tokens,
 * the block-causal keep rule of attends() (:103-109, key-side pad as
 * build_mask :111-142) and the layer calls are the reference's; the layers,
 * projections and final LayerNorm are the loaded model's own objects. Writes
 * the final readout row to out [d]; returns the token count. */
REF_API int ref_octo_forward_layout(void* h, const float* t5, const float* stem_p, const float* stem_w,
                                    int wnd, const uint8_t* tmask, int repeat_task, float* out) {
    auto* t = static_cast<OctoTransformer*>(h);
    const OctoConfig& c = t->cfg;
    const int D = c.d;
    const int rep = repeat_task ? c.n_task : 0;
    const int per = c.tok_primary + c.tok_wrist + rep + c.n_readout;
    const int total = c.n_task + wnd * per;
    std::vector<float> x((size_t)total * D), task((size_t)c.n_task * D);
    t->proj_task.forward(task.data(), t5, c.n_task);
    for (size_t i = 0; i < task.size(); i++) task[i] += t->pos_task[i];
    std::memcpy(x.data(), task.data(), task.size() * sizeof(float));
    // token kinds: 0 task prefix (timestep -1), 1 primary, 2 wrist, 3 repeated task, 4 readout
    std::vector<int> kind(total, 0), step(total, -1);
    std::vector<uint8_t> key_ok(total, 1);
    for (int s = 0; s < wnd; s++) {
        const int base = c.n_task + s * per;
        float* row = x.data() + (size_t)base * D;
        t->proj_prim.forward(row, stem_p + (size_t)s * c.tok_primary * c.stem_dim, c.tok_primary);
        const float* pp = t->pos_prim + (size_t)s * c.tok_primary * D;
        for (size_t i = 0; i < (size_t)c.tok_primary * D; i++) row[i] += pp[i];
        row += (size_t)c.tok_primary * D;
        if (stem_w) {
            t->proj_wrist.forward(row, stem_w + (size_t)s * c.tok_wrist * c.stem_dim, c.tok_wrist);
            const float* pw = t->pos_wrist + (size_t)s * c.tok_wrist * D;
            for (size_t i = 0; i < (size_t)c.tok_wrist * D; i++) row[i] += pw[i];
        }
        row += (size_t)c.tok_wrist * D;
        if (rep) {
            std::memcpy(row, task.data(), task.size() * sizeof(float));
            row += task.size();
        }
        std::memcpy(row, t->pos_readout + (size_t)s * c.n_readout * D, (size_t)c.n_readout * D * sizeof(float));
        for (int i = 0; i < per; i++) {
            const int k = i < c.tok_primary ? 1 : i < c.tok_primary + c.tok_wrist ? 2
                        : i < c.tok_primary + c.tok_wrist + rep ? 3 : 4;
            kind[base + i] = k;
            step[base + i] = s;
            key_ok[base + i] = k == 1 ? tmask[s] != 0 : k == 2 ? (stem_w != nullptr && tmask[s] != 0) : 1;
        }
    }
    const float NEG = std::numeric_limits<float>::lowest();
    std::vector<float> mask((size_t)total * total);
    for (int i = 0; i < total; i++)
        for (int j = 0; j < total; j++) {
            const int gi = kind[i], gj = kind[j], ti = step[i], tj = step[j];
            const bool see = gi == 0 ? gj == 0 : gj == 0 ? true : gj <= 3 ? tj <= ti : (gi == 4 && tj <= ti);
            mask[(size_t)i * total + j] = see && key_ok[j] ? 0.0f : NEG;
        }
    const int ro = c.n_task + wnd * per - 1;
    nn::Scratch s;
    for (size_t li = 0; li + 1 < t->layers.size(); li++) t->layers[li].forward(x.data(), total, mask.data(), s, nullptr);
    t->layers.back().forward_last_row(x.data(), ro, total, mask.data(), s);
    layernorm(out, x.data() + (size_t)ro * D, t->final_s, t->final_b, 1, D, c.ln_eps);
    return total;
}

struct RefSmolvla {
    SmollmVlm vlm;
    ActionExpert aex;
};

REF_API void* ref_smolvla_load(const char* dir, int int8_mask) {
    try {
        const io::Mount mount(dir);
        if (!mount.ok()) return nullptr;
        auto* m = new RefSmolvla();
        if (!m->vlm.load(dir) || !m->aex.load(dir)) {
            delete m;
            return nullptr;
        }
        if (int8_mask & 16)
            for (VlmLayerW& w : m->vlm.layers)
                for (nn::Linear* l : {&w.q, &w.k, &w.v, &w.o, &w.gate, &w.up, &w.down}) l->init_int8();
        if (int8_mask & 32)
            for (ExpertLayerW& w : m->aex.layers)
                for (nn::Linear* l : {&w.q, &w.k, &w.v, &w.o, &w.gate, &w.up, &w.down}) l->init_int8();
        return m;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_smolvla_load: %s\n", e.what());
        return nullptr;
    }
}

/* SmolVLA's SigLIP vision tower + connector (SiglipVision, siglip_vision.cpp),
 * with SmolvlaModel::apply_int8's vision bits (smolvla_model.cpp:49, 127-140):
 * 1 attention, 2 w1, 4 w2, 8 patch embed + modality projection. */
REF_API void* ref_siglip_load(const char* dir, int int8_mask) {
    try {
        const io::Mount mount(dir);
        if (!mount.ok()) return nullptr;
        auto* v = new SiglipVision();
        if (!v->load(dir)) {
            delete v;
            return nullptr;
        }
        for (nn::EncoderLayer& l : v->layers) {
            if (int8_mask & 1) {
                l.attn.wq.init_int8();
                l.attn.wk.init_int8();
                l.attn.wv.init_int8();
                l.attn.wo.init_int8();
            }
            if (int8_mask & 2) l.w1.init_int8();
            if (int8_mask & 4) l.w2.init_int8();
        }
        if (int8_mask & 8) {
            v->patch_lin.init_int8();
            v->mm_proj.init_int8();
        }
        return v;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_siglip_load: %s\n", e.what());
        return nullptr;
    }
}

REF_API void ref_siglip_free(void* h) { delete static_cast<SiglipVision*>(h); }

/* pixels [3, img, img] CHW in [-1, 1] -> out [n_img_tok, mm_out] */
REF_API void ref_siglip_encode(void* h, const float* pixels, float* out) {
    auto* v = static_cast<SiglipVision*>(h);
    nn::Scratch sc;
    v->encode(pixels, out, sc);
}

REF_API void ref_smolvla_free(void* h) { delete static_cast<RefSmolvla*>(h); }

/* prefix [n_prefix, hidden], pad [n_prefix] (last = state token), noise and
 * actions [chunk, max_action_dim] */
REF_API int ref_smolvla_chunk(void* h, const float* prefix, const int* pad, int n_prefix,
                              const float* noise, float* actions) {
    auto* m = static_cast<RefSmolvla*>(h);
    const int C = m->aex.cfg.chunk, np = n_prefix, SK = np + C;
    const float NEG = std::numeric_limits<float>::lowest();
    const int state_idx = np - 1;
    std::vector<float> pmask((size_t)np * np);
    for (int i = 0; i < np; i++)
        for (int j = 0; j < np; j++) {
            const int ai = i >= state_idx, aj = j >= state_idx;
            pmask[(size_t)i * np + j] = (aj <= ai && pad[i] && pad[j]) ? 0.0f : NEG;
        }
    std::vector<int> pos(np);
    int c = 0;
    for (int i = 0; i < np; i++) {  // raw sums, as smolvla_model.cpp:237-238,244
        c += pad[i];
        pos[i] = c - 1;
    }
    std::vector<VlmKV> kv;
    m->vlm.prefix_forward(prefix, pmask.data(), pos.data(), np, kv);
    std::vector<float> dmask((size_t)C * SK);
    std::vector<int> pos_full(C);
    for (int i = 0; i < C; i++) {
        for (int j = 0; j < np; j++) dmask[(size_t)i * SK + j] = pad[j] ? 0.0f : NEG;
        for (int j = 0; j < C; j++) dmask[(size_t)i * SK + np + j] = j <= i ? 0.0f : NEG;
        pos_full[i] = c + i;
    }
    m->aex.denoise(kv, np, noise, dmask.data(), pos_full.data(), actions, nullptr, nullptr, 0.0f);
    return 0;
}

REF_API int ref_smolvla_chunk_len(void* h) { return static_cast<RefSmolvla*>(h)->aex.cfg.chunk; }
REF_API int ref_smolvla_max_action_dim(void* h) {
    return static_cast<RefSmolvla*>(h)->aex.cfg.max_action_dim;
}

/* ActModel (src/models/act/act_model.cpp): load reads ACT_INT8 from the
 * environment as the reference does. dims: chunk, action_dim, state_dim,
 * n_cams, img_h, img_w, feat_h, feat_w, feat_ch. */
REF_API void* ref_act_model_load(const char* dir) {
    try {
        auto* m = new ActModel();
        if (!m->load(dir)) {
            delete m;
            return nullptr;
        }
        return m;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_act_model_load: %s\n", e.what());
        return nullptr;
    }
}

REF_API void ref_act_model_free(void* h) { delete static_cast<ActModel*>(h); }

REF_API void ref_act_model_dims(void* h, int* d) {
    auto* m = static_cast<ActModel*>(h);
    int fh = 0, fw = 0;
    m->backbone.feat_size(m->img_h, m->img_w, &fh, &fw);
    const int v[9] = {m->chunk(), m->action_dim(), m->state_dim(), m->n_cams, m->img_h, m->img_w,
                      fh, fw, m->backbone.out_channels()};
    std::memcpy(d, v, sizeof v);
}

/* images: n_cams uint8 HWC frames back to back (act_capi.cpp:42-53) */
REF_API int ref_act_model_predict(void* h, const uint8_t* images, const float* state, int unnormalize,
                                  float* actions) {
    auto* m = static_cast<ActModel*>(h);
    std::vector<const uint8_t*> ip(m->n_cams);
    for (int c = 0; c < m->n_cams; c++) ip[c] = images + (size_t)c * m->img_h * m->img_w * 3;
    m->predict(ip.data(), state, unnormalize != 0, actions);
    return 0;
}

/* encode_view per camera: feats [n_cams, fh * fw, ch] */
REF_API int ref_act_model_encode(void* h, const uint8_t* images, float* feats) {
    auto* m = static_cast<ActModel*>(h);
    int fh = 0, fw = 0;
    m->backbone.feat_size(m->img_h, m->img_w, &fh, &fw);
    const size_t nf = (size_t)fh * fw * m->backbone.out_channels();
    for (int c = 0; c < m->n_cams; c++)
        m->encode_view(images + (size_t)c * m->img_h * m->img_w * 3, c, feats + (size_t)c * nf);
    return 0;
}

/* SmolvlaModel::load, then SmolvlaModel::apply_int8's groups for int8_mask
 * (smolvla_model.cpp:111-155). The caller leaves SMOLVLA_INT8 unset so that
 * load's own apply_int8 quantizes nothing. */
REF_API void* ref_smolvla_model_load(const char* dir, int int8_mask) {
    try {
        const io::Mount mount(dir);
        if (!mount.ok()) return nullptr;
        auto* m = new SmolvlaModel();
        if (!m->load(dir)) {
            delete m;
            return nullptr;
        }
        for (nn::EncoderLayer& l : m->vit.layers) {
            if (int8_mask & 1)
                for (nn::Linear* x : {&l.attn.wq, &l.attn.wk, &l.attn.wv, &l.attn.wo}) x->init_int8();
            if (int8_mask & 2) l.w1.init_int8();
            if (int8_mask & 4) l.w2.init_int8();
        }
        if (int8_mask & 8) {
            m->vit.patch_lin.init_int8();
            m->vit.mm_proj.init_int8();
        }
        if (int8_mask & 16)
            for (VlmLayerW& w : m->vlm.layers)
                for (nn::Linear* l : {&w.q, &w.k, &w.v, &w.o, &w.gate, &w.up, &w.down}) l->init_int8();
        if (int8_mask & 32)
            for (ExpertLayerW& w : m->aex.layers)
                for (nn::Linear* l : {&w.q, &w.k, &w.v, &w.o, &w.gate, &w.up, &w.down}) l->init_int8();
        return m;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_smolvla_model_load: %s\n", e.what());
        return nullptr;
    }
}

REF_API void ref_smolvla_model_free(void* h) { delete static_cast<SmolvlaModel*>(h); }

/* vla_smolvla_predict_rtc's body (smolvla_capi.cpp:146-166) with the noise
 * given: resize_with_pad per view, SmolvlaModel::predict, the first
 * real_action_dim columns of each row. Returns 0, or -2 when predict rejects
 * the input. perturb > 0 moves every preprocessed pixel by -1, 0 or +1 ulp
 * (a xorshift stream seeded by perturb) before the model sees it: the class
 * of difference an fp32 vision tower's summation order leaves, for the tests'
 * sensitivity bars. */
REF_API int ref_smolvla_model_predict(void* h, const uint8_t* frames, int nv, int height, int width,
                                      const int32_t* tokens, const int32_t* lmask, int n_lang, const float* state,
                                      const float* noise, float* actions, const float* prev, int n_prev,
                                      const float* weights, float max_guidance, int perturb) {
    const auto& m = *static_cast<SmolvlaModel*>(h);
    const int S = m.vit.cfg.img, C = m.aex.cfg.chunk, MAD = m.aex.cfg.max_action_dim;
    const size_t per_view = (size_t)3 * S * S;
    std::vector<float> pixels((size_t)nv * per_view);
    for (int v = 0; v < nv; v++)
        resize_with_pad(frames + (size_t)v * height * width * 3, height, width, S, pixels.data() + (size_t)v * per_view);
    if (perturb > 0) {
        uint64_t x = 0x9E3779B97F4A7C15ull * (uint64_t)perturb;
        for (float& p : pixels) {
            x ^= x << 13;
            x ^= x >> 7;
            x ^= x << 17;
            const int d = (int)(x % 3) - 1;
            if (d) p = std::nextafter(p, d > 0 ? INFINITY : -INFINITY);
        }
    }
    auto out = m.predict(pixels.data(), nv, tokens, lmask, n_lang, state, noise, prev, n_prev, weights, max_guidance);
    if (out.empty()) return -2;
    for (int t = 0; t < C; t++)
        std::memcpy(actions + (size_t)t * m.real_action_dim, out.data() + (size_t)t * MAD,
                    m.real_action_dim * sizeof(float));
    return 0;
}

REF_API void ref_resize_with_pad(const uint8_t* src, int h, int w, int S, float* dst) {
    resize_with_pad(src, h, w, S, dst);
}

REF_API void* ref_bpe_load(const char* dir) {
    try {
        auto* t = new Tokenizer();
        if (!t->load(dir)) {
            delete t;
            return nullptr;
        }
        return t;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_bpe_load: %s\n", e.what());
        return nullptr;
    }
}
REF_API void ref_bpe_free(void* h) { delete static_cast<Tokenizer*>(h); }
/* Tokenizer::encode: writes at most cap ids, returns the count */
REF_API int ref_bpe_encode(void* h, const char* text, int32_t* ids, int cap) {
    const std::vector<int> v = static_cast<Tokenizer*>(h)->encode(text);
    for (int i = 0; i < (int)v.size() && i < cap; i++) ids[i] = v[i];
    return (int)v.size();
}

REF_API void* ref_t5tok_load(const char* dir) {
    try {
        auto* t = new T5Tokenizer();
        if (!t->load(dir)) {
            delete t;
            return nullptr;
        }
        return t;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_t5tok_load: %s\n", e.what());
        return nullptr;
    }
}
REF_API void ref_t5tok_free(void* h) { delete static_cast<T5Tokenizer*>(h); }
/* T5Tokenizer::encode(text, max_len): max_len ids */
REF_API void ref_t5tok_encode(void* h, const char* text, int max_len, int32_t* ids) {
    const std::vector<int> v = static_cast<T5Tokenizer*>(h)->encode(text, max_len);
    for (int i = 0; i < (int)v.size(); i++) ids[i] = v[i];
}

/* OctoModel::load, then OctoModel::apply_int8's groups for int8_mask. The
 * caller leaves OCTO_INT8 unset so that load's own apply_int8 does nothing. */
REF_API void* ref_octo_model_load(const char* dir, const char* tok_dir, int int8_mask) {
    try {
        auto* m = new OctoModel();
        if (!m->load(dir, tok_dir)) {
            delete m;
            return nullptr;
        }
        for (nn::EncoderLayer& l : m->tf.layers) {
            if (int8_mask & 1)
                for (nn::Linear* x : {&l.attn.wq, &l.attn.wk, &l.attn.wv, &l.attn.wo}) x->init_int8();
            if (int8_mask & 2) l.w1.init_int8();
            if (int8_mask & 4) l.w2.init_int8();
        }
        if (int8_mask & 8)
            for (nn::Linear* x : {&m->tf.proj_task, &m->tf.proj_prim, &m->tf.proj_wrist, &m->stem_primary.embed,
                                  &m->stem_wrist.embed})
                x->init_int8();
        if (int8_mask & 16)
            for (SmallStem* st : {&m->stem_primary, &m->stem_wrist})
                for (StemLayer& l : st->layers) l.conv.init_int8();
        if (int8_mask & 32) {
            m->head.net.in_proj.init_int8();
            m->head.net.out_proj.init_int8();
            for (nn::DiffusionMlp::Block& b : m->head.net.blocks) {
                b.d0.init_int8();
                b.d1.init_int8();
            }
        }
        return m;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_octo_model_load: %s\n", e.what());
        return nullptr;
    }
}

REF_API void ref_octo_model_free(void* h) { delete static_cast<OctoModel*>(h); }

/* horizon, action_dim, max_window, n_task, t5_dim, steps */
REF_API void ref_octo_model_dims(void* h, int* d) {
    const auto& m = *static_cast<OctoModel*>(h);
    d[0] = m.head.cfg.horizon;
    d[1] = m.head.cfg.action_dim;
    d[2] = m.tf.cfg.max_horizon;
    d[3] = m.tf.cfg.n_task;
    d[4] = m.t5.cfg.d_model;
    d[5] = m.head.cfg.steps;
}

/* OctoModel::lang_encode's value: [n_task, d_model] */
REF_API void ref_octo_model_lang(void* h, const char* instruction, float* out) {
    const auto& m = *static_cast<OctoModel*>(h);
    const int NT = m.tf.cfg.n_task;
    std::vector<int> ids = m.tok.encode(instruction, NT);
    std::vector<int> am(NT);
    for (int i = 0; i < NT; i++) am[i] = ids[i] != m.tok.pad_id;
    m.t5.encode(ids.data(), am.data(), NT, out);
}

/* OctoModel::predict with the noise given; perturb > 0 moves every stem token
 * value by -1, 0 or +1 ulp (xorshift seeded by perturb): the class of
 * difference fp32 stem convolutions with another summation order leave. */
REF_API void ref_octo_model_predict(void* h, const uint8_t* primary, const uint8_t* wrist, int wnd,
                                    const uint8_t* tmask, const char* instruction, const float* noise, const float* z,
                                    int unnormalize, float* actions, int perturb) {
    const auto& m = *static_cast<OctoModel*>(h);
    const int D = m.tf.cfg.d;
    const size_t PB = (size_t)256 * 256 * 3, WB = (size_t)128 * 128 * 3;
    const size_t SP = (size_t)m.tf.cfg.tok_primary * m.tf.cfg.stem_dim, SW = (size_t)m.tf.cfg.tok_wrist * m.tf.cfg.stem_dim;
    std::vector<float> sp((size_t)wnd * SP), sw(wrist ? (size_t)wnd * SW : 0);
    for (int t = 0; t < wnd; t++) {
        m.stem_primary.encode(primary + (size_t)t * PB, 256, 256, sp.data() + (size_t)t * SP);
        if (wrist) m.stem_wrist.encode(wrist + (size_t)t * WB, 128, 128, sw.data() + (size_t)t * SW);
    }
    if (perturb > 0) {
        uint64_t x = 0x9E3779B97F4A7C15ull * (uint64_t)perturb;
        for (std::vector<float>* v : {&sp, &sw})
            for (float& p : *v) {
                x ^= x << 13;
                x ^= x >> 7;
                x ^= x << 17;
                const int d = (int)(x % 3) - 1;
                if (d) p = std::nextafter(p, d > 0 ? INFINITY : -INFINITY);
            }
    }
    const int NT = m.tf.cfg.n_task;
    std::vector<float> t5((size_t)NT * m.t5.cfg.d_model);
    ref_octo_model_lang(h, instruction, t5.data());
    std::vector<float> out((size_t)m.tf.total_tokens(wnd) * D);
    m.tf.forward(t5.data(), sp.data(), wrist ? sw.data() : nullptr, wnd, tmask, out.data());
    const float* emb = out.data() + (size_t)m.tf.readout_index(wnd, wnd - 1) * D;
    m.head.denoise(emb, noise, z, actions);
    if (unnormalize)
        for (int hh = 0; hh < m.head.cfg.horizon; hh++)
            for (int a = 0; a < m.head.cfg.action_dim; a++) {
                float* v = actions + (size_t)hh * m.head.cfg.action_dim + a;
                if (m.act_mask[a] > 0.0f) *v = *v * m.act_std[a] + m.act_mean[a];
            }
}
