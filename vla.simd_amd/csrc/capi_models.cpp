// capi_models.cpp - extern "C" entry points of the device policy graphs
// (models.h). Handles own their weights, buffers, stream and captured graph;
// one inference per handle at a time (include/vla_simd.h:22-25). Host-pointer
// forms upload, run on a private stream and synchronize; _dev forms take
// device pointers and a hipStream_t and return without waiting.

#include "vla_simd_hip.h"

#include "ckpt.h"
#include "models.h"
#include "runtime.h"

#include <cstdio>
#include <cstring>
#include <memory>

using namespace vla::hip;

struct vla_ckpt {
    std::unique_ptr<CkptFiles> f;
};
struct vla_act_tf {
    std::unique_ptr<ActTf> m;
};
struct vla_octo_tf {
    std::unique_ptr<OctoTf> m;
};
struct vla_smolvla_tf {
    std::unique_ptr<SmolvlaTf> m;
};
struct vla_siglip_tf {
    std::unique_ptr<SiglipTf> m;
};

namespace {

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// Upload / run / download on a private stream for the host-pointer forms.
struct HostCall {
    hipStream_t st = nullptr;
    std::vector<void*> bufs;
    HostCall() { VLA_HIP_CHECK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking)); }
    ~HostCall() {
        if (st) (void)hipStreamSynchronize(st);
        for (void* p : bufs) (void)hipFree(p);
        if (st) (void)hipStreamDestroy(st);
    }
    void* raw(size_t bytes) {
        void* p = nullptr;
        VLA_HIP_CHECK(hipMalloc(&p, bytes ? bytes : 16));
        bufs.push_back(p);
        return p;
    }
    template <class T>
    T* up(const T* h, size_t n) {
        if (!h) return nullptr;
        T* p = static_cast<T*>(raw(n * sizeof(T)));
        VLA_HIP_CHECK(hipMemcpyAsync(p, h, n * sizeof(T), hipMemcpyHostToDevice, st));
        return p;
    }
    float* out(size_t n) { return static_cast<float*>(raw(n * 4)); }
    void down(float* h, const float* d, size_t n) {
        VLA_HIP_CHECK(hipMemcpyAsync(h, d, n * 4, hipMemcpyDeviceToHost, st));
        VLA_HIP_CHECK(hipStreamSynchronize(st));
    }
};

template <class H, class F>
H* load_handle(const char* where, F&& make) {
    H* h = nullptr;
    const int32_t rc = guarded(where, [&] {
        auto p = std::make_unique<H>();
        p->m = make();
        h = p.release();
    });
    return rc == 0 ? h : nullptr;
}

}  // namespace

extern "C" {

// ------------------------------------------------------ checkpoint files --

VLA_API vla_ckpt* vla_ckpt_open(const char* path) {
    vla_ckpt* h = nullptr;
    const int32_t rc = guarded("vla_ckpt_open", [&] {
        VLA_REQUIRE(path, "null path");
        auto p = std::make_unique<vla_ckpt>();
        p->f = std::make_unique<CkptFiles>(path);
        h = p.release();
    });
    return rc == 0 ? h : nullptr;
}

VLA_API void vla_ckpt_free(vla_ckpt* c) { delete c; }

VLA_API int32_t vla_ckpt_is_gguf(const vla_ckpt* c) { return c && c->f->gguf() ? 1 : 0; }

VLA_API int64_t vla_ckpt_file_size(const vla_ckpt* c, const char* rel) {
    if (!c || !rel) return -1;
    int64_t n = -1;
    (void)guarded("vla_ckpt_file_size", [&] { n = c->f->size(rel); });
    return n;
}

VLA_API int32_t vla_ckpt_read(const vla_ckpt* c, const char* rel, void* buf, int64_t cap) {
    return guarded("vla_ckpt_read", [&] {
        VLA_REQUIRE(c && rel, "null handle or name");
        const std::vector<char> d = c->f->bytes(rel);
        VLA_REQUIRE((int64_t)d.size() <= cap && (buf || d.empty()), "buffer too small");
        if (!d.empty()) std::memcpy(buf, d.data(), d.size());
    });
}

VLA_API int64_t vla_ckpt_names(const vla_ckpt* c, char* buf, int64_t cap) {
    if (!c) return -1;
    std::string all;
    for (const std::string& n : c->f->names()) {
        if (!all.empty()) all += '\n';
        all += n;
    }
    const int64_t need = (int64_t)all.size() + 1;
    if (buf && cap >= need) std::memcpy(buf, all.c_str(), (size_t)need);
    return need;
}

// ------------------------------------------------------------------- ACT --

VLA_API vla_act_tf* vla_act_tf_load(const char* dir, int32_t img_ch, int32_t int8_mask) {
    return load_handle<vla_act_tf>("vla_act_tf_load", [&] {
        VLA_REQUIRE(dir, "null directory");
        return std::make_unique<ActTf>(dir, img_ch, int8_mask);
    });
}
VLA_API void vla_act_tf_free(vla_act_tf* h) { delete h; }
VLA_API int32_t vla_act_tf_chunk(const vla_act_tf* h) { return h ? h->m->chunk() : 0; }
VLA_API int32_t vla_act_tf_action_dim(const vla_act_tf* h) { return h ? h->m->action_dim() : 0; }
VLA_API int32_t vla_act_tf_state_dim(const vla_act_tf* h) { return h ? h->m->state_dim() : 0; }
VLA_API int32_t vla_act_tf_dim(const vla_act_tf* h) { return h ? h->m->dim() : 0; }
VLA_API int32_t vla_act_tf_int8_layers(const vla_act_tf* h) { return h ? h->m->int8_layers() : 0; }
VLA_API int32_t vla_act_tf_graph_nodes(const vla_act_tf* h) { return h ? h->m->graph_nodes() : 0; }

VLA_API int32_t vla_act_tf_forward_dev(vla_act_tf* h, const float* feats, int32_t n_cams, int32_t fh,
                                       int32_t fw, const float* state_norm, float* actions_norm,
                                       void* stream) {
    return guarded("vla_act_tf_forward_dev", [&] {
        VLA_REQUIRE(h, "null handle");
        h->m->forward_dev(feats, n_cams, fh, fw, state_norm, actions_norm, as_stream(stream));
    });
}

VLA_API int32_t vla_act_tf_forward(vla_act_tf* h, const float* feats, int32_t n_cams, int32_t fh,
                                   int32_t fw, const float* state_norm, float* actions_norm) {
    return guarded("vla_act_tf_forward", [&] {
        VLA_REQUIRE(h && feats && state_norm && actions_norm, "null handle or buffer");
        VLA_REQUIRE(n_cams > 0 && fh > 0 && fw > 0, "camera grid out of range");
        ActTf& m = *h->m;
        HostCall hc;
        const float* df = hc.up(feats, (size_t)n_cams * fh * fw * m.img_ch());
        const float* ds = hc.up(state_norm, (size_t)m.state_dim());
        const size_t na = (size_t)m.chunk() * m.action_dim();
        float* da = hc.out(na);
        m.forward_dev(df, n_cams, fh, fw, ds, da, hc.st);
        hc.down(actions_norm, da, na);
    });
}

VLA_API vla_act_tf* vla_act_tf_load_ex(const char* dir, int32_t img_ch, int32_t int8_mask, int32_t int8_state) {
    return load_handle<vla_act_tf>("vla_act_tf_load_ex", [&] {
        VLA_REQUIRE(dir, "null directory");
        return std::make_unique<ActTf>(dir, img_ch, int8_mask, int8_state != 0);
    });
}
VLA_API int32_t vla_act_tf_n_text(const vla_act_tf* h) { return h ? h->m->n_text() : 0; }

VLA_API int32_t vla_act_tf_forward_text_dev(vla_act_tf* h, const float* feats, int32_t n_cams, int32_t fh,
                                            int32_t fw, const float* state_norm, const float* text,
                                            const float* text_pos, int32_t n_text_real, float* actions_norm,
                                            void* stream) {
    return guarded("vla_act_tf_forward_text_dev", [&] {
        VLA_REQUIRE(h, "null handle");
        h->m->forward_text_dev(feats, n_cams, fh, fw, state_norm, text, text_pos, n_text_real, actions_norm,
                               as_stream(stream));
    });
}

VLA_API int32_t vla_act_tf_forward_text(vla_act_tf* h, const float* feats, int32_t n_cams, int32_t fh, int32_t fw,
                                        const float* state_norm, const float* text, const float* text_pos,
                                        int32_t n_text_real, float* actions_norm) {
    return guarded("vla_act_tf_forward_text", [&] {
        VLA_REQUIRE(h && feats && state_norm && actions_norm, "null handle or buffer");
        VLA_REQUIRE(n_cams > 0 && fh > 0 && fw > 0, "camera grid out of range");
        ActTf& m = *h->m;
        const int nt = n_text_real < 0 ? 0 : n_text_real > m.n_text() ? m.n_text() : n_text_real;
        VLA_REQUIRE(nt == 0 || (text && text_pos), "text tokens without their positions");
        HostCall hc;
        const float* df = hc.up(feats, (size_t)n_cams * fh * fw * m.img_ch());
        const float* ds = hc.up(state_norm, (size_t)m.state_dim());
        const float* dt = nt ? hc.up(text, (size_t)nt * m.dim()) : nullptr;
        const float* dp = nt ? hc.up(text_pos, (size_t)nt * m.dim()) : nullptr;
        const size_t na = (size_t)m.chunk() * m.action_dim();
        float* da = hc.out(na);
        m.forward_text_dev(df, n_cams, fh, fw, ds, dt, dp, nt, da, hc.st);
        hc.down(actions_norm, da, na);
    });
}

// ------------------------------------------------------------------ Octo --

VLA_API vla_octo_tf* vla_octo_tf_load(const char* dir, int32_t int8_mask) {
    return load_handle<vla_octo_tf>("vla_octo_tf_load", [&] {
        VLA_REQUIRE(dir, "null directory");
        return std::make_unique<OctoTf>(dir, int8_mask);
    });
}
VLA_API void vla_octo_tf_free(vla_octo_tf* h) { delete h; }
VLA_API int32_t vla_octo_tf_dim(const vla_octo_tf* h) { return h ? h->m->d() : 0; }
VLA_API int32_t vla_octo_tf_total_tokens(const vla_octo_tf* h, int32_t wnd) {
    return h ? h->m->total_tokens(wnd) : 0;
}
VLA_API int32_t vla_octo_tf_config(const vla_octo_tf* h, int32_t* cfg) {
    return guarded("vla_octo_tf_config", [&] {
        VLA_REQUIRE(h && cfg, "null handle or buffer");
        const OctoTf& m = *h->m;
        const int32_t v[7] = {m.d(), m.n_task(), m.t5_dim(), m.stem_dim(), m.tok_primary(), m.tok_wrist(),
                              m.max_horizon()};
        std::memcpy(cfg, v, sizeof v);
    });
}

VLA_API int32_t vla_octo_tf_readout_index(const vla_octo_tf* h, int32_t wnd) {
    return h ? h->m->readout_index(wnd) : 0;
}
VLA_API int32_t vla_octo_tf_int8_layers(const vla_octo_tf* h) { return h ? h->m->int8_layers() : 0; }
VLA_API int32_t vla_octo_tf_graph_nodes(const vla_octo_tf* h) { return h ? h->m->graph_nodes() : 0; }

VLA_API int32_t vla_octo_tf_forward_dev(vla_octo_tf* h, const float* t5_out, const float* stem_p,
                                        const float* stem_w, int32_t wnd, const uint8_t* timestep_mask,
                                        float* out, void* stream) {
    return guarded("vla_octo_tf_forward_dev", [&] {
        VLA_REQUIRE(h, "null handle");
        h->m->forward_dev(t5_out, stem_p, stem_w, wnd, timestep_mask, out, as_stream(stream));
    });
}

VLA_API int32_t vla_octo_tf_forward(vla_octo_tf* h, const float* t5_out, const float* stem_p,
                                    const float* stem_w, int32_t wnd, const uint8_t* timestep_mask,
                                    float* out) {
    return guarded("vla_octo_tf_forward", [&] {
        VLA_REQUIRE(h && t5_out && stem_p && timestep_mask && out, "null handle or buffer");
        OctoTf& m = *h->m;
        VLA_REQUIRE(wnd >= 1 && wnd <= m.max_horizon(), "window must be in [1, max_horizon]");
        HostCall hc;
        const float* dt = hc.up(t5_out, (size_t)m.n_task() * m.t5_dim());
        const float* dp = hc.up(stem_p, (size_t)wnd * m.tok_primary() * m.stem_dim());
        const float* dw = stem_w ? hc.up(stem_w, (size_t)wnd * m.tok_wrist() * m.stem_dim()) : nullptr;
        float* dout = hc.out((size_t)m.d());
        m.forward_dev(dt, dp, dw, wnd, timestep_mask, dout, hc.st);
        hc.down(out, dout, (size_t)m.d());
    });
}

// --------------------------------------------------------------- SmolVLA --

VLA_API vla_smolvla_tf* vla_smolvla_tf_load(const char* dir, int32_t int8_mask) {
    return load_handle<vla_smolvla_tf>("vla_smolvla_tf_load", [&] {
        VLA_REQUIRE(dir, "null directory");
        return std::make_unique<SmolvlaTf>(dir, int8_mask);
    });
}
VLA_API void vla_smolvla_tf_free(vla_smolvla_tf* h) { delete h; }
VLA_API int32_t vla_smolvla_tf_chunk(const vla_smolvla_tf* h) { return h ? h->m->chunk() : 0; }
VLA_API int32_t vla_smolvla_tf_max_action_dim(const vla_smolvla_tf* h) {
    return h ? h->m->max_action_dim() : 0;
}
VLA_API int32_t vla_smolvla_tf_hidden(const vla_smolvla_tf* h) { return h ? h->m->hidden() : 0; }
VLA_API int32_t vla_smolvla_tf_int8_layers(const vla_smolvla_tf* h) { return h ? h->m->int8_layers() : 0; }
VLA_API int32_t vla_smolvla_tf_graph_nodes(const vla_smolvla_tf* h) { return h ? h->m->graph_nodes() : 0; }

VLA_API int32_t vla_smolvla_tf_chunk_dev(vla_smolvla_tf* h, const float* prefix, const int32_t* pad,
                                         int32_t n_prefix, const float* noise, float* actions,
                                         void* stream) {
    return guarded("vla_smolvla_tf_chunk_dev", [&] {
        VLA_REQUIRE(h, "null handle");
        h->m->chunk_dev(prefix, pad, n_prefix, noise, actions, as_stream(stream));
    });
}

VLA_API int32_t vla_smolvla_tf_chunk_run(vla_smolvla_tf* h, const float* prefix, const int32_t* pad,
                                         int32_t n_prefix, const float* noise, float* actions) {
    return guarded("vla_smolvla_tf_chunk_run", [&] {
        VLA_REQUIRE(h && prefix && pad && noise && actions, "null handle or buffer");
        VLA_REQUIRE(n_prefix >= 2, "prefix too short");
        SmolvlaTf& m = *h->m;
        HostCall hc;
        const float* dp = hc.up(prefix, (size_t)n_prefix * m.hidden());
        const size_t na = (size_t)m.chunk() * m.max_action_dim();
        const float* dn = hc.up(noise, na);
        float* da = hc.out(na);
        m.chunk_dev(dp, pad, n_prefix, dn, da, hc.st);
        hc.down(actions, da, na);
    });
}

}  // extern "C"

// ---------------------------------------------------------------- SigLIP --

VLA_API vla_siglip_tf* vla_siglip_tf_load(const char* dir, int32_t int8_mask) {
    return load_handle<vla_siglip_tf>("vla_siglip_tf_load", [&] {
        VLA_REQUIRE(dir, "null directory");
        return std::make_unique<SiglipTf>(dir, int8_mask);
    });
}
VLA_API void vla_siglip_tf_free(vla_siglip_tf* h) { delete h; }
VLA_API int32_t vla_siglip_tf_img(const vla_siglip_tf* h) { return h ? h->m->img() : 0; }
VLA_API int32_t vla_siglip_tf_n_tokens(const vla_siglip_tf* h) { return h ? h->m->n_tokens() : 0; }
VLA_API int32_t vla_siglip_tf_out_dim(const vla_siglip_tf* h) { return h ? h->m->out_dim() : 0; }
VLA_API int32_t vla_siglip_tf_int8_layers(const vla_siglip_tf* h) { return h ? h->m->int8_layers() : 0; }
VLA_API int32_t vla_siglip_tf_graph_nodes(const vla_siglip_tf* h) { return h ? h->m->graph_nodes() : 0; }

VLA_API int32_t vla_siglip_tf_encode_dev(vla_siglip_tf* h, const float* pixels, float* out, void* stream) {
    return guarded("vla_siglip_tf_encode_dev", [&] {
        VLA_REQUIRE(h, "null handle");
        h->m->encode_dev(pixels, out, as_stream(stream));
    });
}

VLA_API int32_t vla_siglip_tf_encode(vla_siglip_tf* h, const float* pixels, float* out) {
    return guarded("vla_siglip_tf_encode", [&] {
        VLA_REQUIRE(h && pixels && out, "null handle or buffer");
        SiglipTf& m = *h->m;
        HostCall hc;
        const float* dp = hc.up(pixels, (size_t)3 * m.img() * m.img());
        const size_t n = (size_t)m.n_tokens() * m.out_dim();
        float* dout = hc.out(n);
        m.encode_dev(dp, dout, hc.st);
        hc.down(out, dout, n);
    });
}

// ----------------------------------------------------------------- probe --

VLA_API int32_t vla_probe_begin(int32_t max_records) {
    return guarded("vla_probe_begin", [&] {
        VLA_REQUIRE(max_records >= 0, "max_records must be >= 0");
        probe_begin(max_records);
    });
}

VLA_API int32_t vla_probe_end(void) {
    return guarded("vla_probe_end", [&] { probe_end(); });
}

VLA_API int32_t vla_probe_count(void) { return (int32_t)probe_records().size(); }

VLA_API int32_t vla_probe_shape(int32_t i, int32_t* shape) {
    return guarded("vla_probe_shape", [&] {
        const auto& R = probe_records();
        VLA_REQUIRE(i >= 0 && (size_t)i < R.size() && shape, "record index out of range or null shape");
        const ProbeRecord& r = R[i];
        const int32_t v[7] = {r.M, r.K, r.N, r.act, r.acc, r.has_bias, r.has_src};
        std::memcpy(shape, v, sizeof v);
    });
}

VLA_API int32_t vla_probe_read(int32_t i, int32_t what, void* dst, int64_t bytes) {
    return guarded("vla_probe_read", [&] {
        const auto& R = probe_records();
        VLA_REQUIRE(i >= 0 && (size_t)i < R.size() && dst, "record index out of range or null buffer");
        const ProbeRecord& r = R[i];
        const void* src = nullptr;
        size_t n = 0;
        switch (what) {
        case VLA_PROBE_SRC: src = r.src.data(); n = r.src.size() * 4; break;
        case VLA_PROBE_XQ: src = r.xq.data(); n = r.xq.size(); break;
        case VLA_PROBE_ASCALE: src = r.as.data(); n = r.as.size() * 4; break;
        case VLA_PROBE_BEFORE: src = r.before.data(); n = r.before.size() * 4; break;
        case VLA_PROBE_AFTER: src = r.after.data(); n = r.after.size() * 4; break;
        case VLA_PROBE_W: src = r.W.data(); n = r.W.size(); break;
        case VLA_PROBE_WSCALE: src = r.ws.data(); n = r.ws.size() * 4; break;
        case VLA_PROBE_BIAS: src = r.bias.data(); n = r.bias.size() * 4; break;
        default: throw ArgError("unknown probe field");
        }
        VLA_REQUIRE(bytes == (int64_t)n, "buffer size does not match the field");
        if (n) std::memcpy(dst, src, n);
    });
}

// ------------------------------------------------------ ACT (model level) --
// The reference's own ACT entry points (include/vla_simd.h:66-81,
// src/models/act/act_capi.cpp): void* handles, 0 from the accessors on a null
// handle, VLA_ERR_ARG for null buffers, exceptions as VLA_ERR_EXCEPTION.

namespace {
ActModel* act_model(void* h) { return static_cast<ActModel*>(h); }
}  // namespace

VLA_API void* vla_act_load(const char* model_dir) {
    ActModel* m = nullptr;
    const int32_t rc = guarded("vla_act_load", [&] {
        VLA_REQUIRE(model_dir, "null model directory");
        m = new ActModel(model_dir);
    });
    return rc == 0 ? m : nullptr;
}
VLA_API void vla_act_free(void* h) { delete act_model(h); }
VLA_API int32_t vla_act_chunk(void* h) { return h ? act_model(h)->chunk() : 0; }
VLA_API int32_t vla_act_action_dim(void* h) { return h ? act_model(h)->action_dim() : 0; }
VLA_API int32_t vla_act_state_dim(void* h) { return h ? act_model(h)->state_dim() : 0; }
VLA_API int32_t vla_act_n_cams(void* h) { return h ? act_model(h)->n_cams() : 0; }
VLA_API int32_t vla_act_img_h(void* h) { return h ? act_model(h)->img_h() : 0; }
VLA_API int32_t vla_act_img_w(void* h) { return h ? act_model(h)->img_w() : 0; }
VLA_API int32_t vla_act_int8_convs(void* h) { return h ? act_model(h)->int8_convs() : 0; }
VLA_API int32_t vla_act_int8_layers(void* h) { return h ? act_model(h)->int8_layers() : 0; }
VLA_API int32_t vla_act_graph_nodes(void* h) { return h ? act_model(h)->graph_nodes() : 0; }
VLA_API int32_t vla_act_feat_shape(void* h, int32_t* fh, int32_t* fw, int32_t* ch) {
    return guarded("vla_act_feat_shape", [&] {
        VLA_REQUIRE(h && fh && fw && ch, "null handle or buffer");
        *fh = act_model(h)->feat_h();
        *fw = act_model(h)->feat_w();
        *ch = act_model(h)->feat_ch();
    });
}

VLA_API int32_t vla_act_predict(void* h, const uint8_t* images, const float* state, int32_t unnormalize,
                                float* actions) {
    if (!h || !images || !state || !actions) return VLA_ERR_ARG;
    return guarded("vla_act_predict", [&] {
        ActModel& m = *act_model(h);
        HostCall hc;
        const size_t nimg = (size_t)m.n_cams() * m.img_h() * m.img_w() * 3;
        const uint8_t* di = hc.up(images, nimg);
        const float* ds = hc.up(state, (size_t)m.state_dim());
        const size_t na = (size_t)m.chunk() * m.action_dim();
        float* da = hc.out(na);
        m.predict_dev(di, ds, unnormalize != 0, da, hc.st);
        hc.down(actions, da, na);
    });
}

VLA_API int32_t vla_act_predict_dev(void* h, const uint8_t* images, const float* state, int32_t unnormalize,
                                    float* actions, void* stream) {
    if (!h || !images || !state || !actions) return VLA_ERR_ARG;
    return guarded("vla_act_predict_dev", [&] {
        act_model(h)->predict_dev(images, state, unnormalize != 0, actions, as_stream(stream));
    });
}

VLA_API int32_t vla_act_encode(void* h, const uint8_t* images, float* feats) {
    if (!h || !images || !feats) return VLA_ERR_ARG;
    return guarded("vla_act_encode", [&] {
        ActModel& m = *act_model(h);
        HostCall hc;
        const uint8_t* di = hc.up(images, (size_t)m.n_cams() * m.img_h() * m.img_w() * 3);
        const size_t nf = (size_t)m.n_cams() * m.feat_h() * m.feat_w() * m.feat_ch();
        float* df = hc.out(nf);
        m.encode_dev(di, df, hc.st);
        hc.down(feats, df, nf);
    });
}

VLA_API int32_t vla_act_encode_dev(void* h, const uint8_t* images, float* feats, void* stream) {
    if (!h || !images || !feats) return VLA_ERR_ARG;
    return guarded("vla_act_encode_dev", [&] { act_model(h)->encode_dev(images, feats, as_stream(stream)); });
}

// --------------------------------------------------- IMPACT (model level) --
// The reference's IMPACT entry points (include/vla_simd.h:206-243,
// src/models/impact/impact_capi.cpp), same names, signatures and status codes.

namespace {
ImpactModel* impact_model(void* h) { return static_cast<ImpactModel*>(h); }
}  // namespace

VLA_API void* vla_impact_load(const char* model_dir) {
    ImpactModel* m = nullptr;
    const int32_t rc = guarded("vla_impact_load", [&] {
        VLA_REQUIRE(model_dir, "null model directory");
        m = new ImpactModel(model_dir);
    });
    return rc == 0 ? m : nullptr;
}
VLA_API void vla_impact_free(void* h) { delete impact_model(h); }
VLA_API int32_t vla_impact_chunk(void* h) { return h ? impact_model(h)->chunk() : 0; }
VLA_API int32_t vla_impact_action_dim(void* h) { return h ? impact_model(h)->action_dim() : 0; }
VLA_API int32_t vla_impact_state_dim(void* h) { return h ? impact_model(h)->state_dim() : 0; }
VLA_API int32_t vla_impact_n_cams(void* h) { return h ? impact_model(h)->n_cams() : 0; }
VLA_API int32_t vla_impact_img_h(void* h) { return h ? impact_model(h)->img_h() : 0; }
VLA_API int32_t vla_impact_img_w(void* h) { return h ? impact_model(h)->img_w() : 0; }
VLA_API int32_t vla_impact_n_text(void* h) { return h ? impact_model(h)->n_text() : 0; }
VLA_API int32_t vla_impact_int8_layers(void* h) { return h ? impact_model(h)->int8_layers() : 0; }
VLA_API int32_t vla_impact_int8_convs(void* h) { return h ? impact_model(h)->int8_convs() : 0; }

VLA_API int32_t vla_impact_set_instruction(void* h, const char* instruction) {
    if (!h || !instruction) return VLA_ERR_ARG;
    const int32_t rc = guarded("vla_impact_set_instruction", [&] { impact_model(h)->set_instruction(instruction); });
    return rc == 0 ? VLA_OK : VLA_ERR_EXCEPTION;  // impact_capi.cpp:46-51: anything thrown is an exception
}

VLA_API int32_t vla_impact_predict(void* h, const uint8_t* frames, const float* state, const char* instruction,
                                   int32_t unnormalize, float* actions) {
    if (!h || !frames || !state || !instruction || !actions) return VLA_ERR_ARG;
    const int32_t rc = guarded("vla_impact_predict", [&] {
        ImpactModel& m = *impact_model(h);
        m.set_instruction(instruction);
        HostCall hc;
        const size_t nimg = (size_t)m.n_cams() * m.img_h() * m.img_w() * 3;
        const uint8_t* di = hc.up(frames, nimg);
        const float* ds = hc.up(state, (size_t)m.state_dim());
        const size_t na = (size_t)m.chunk() * m.action_dim();
        float* da = hc.out(na);
        m.predict_dev(di, ds, unnormalize != 0, da, hc.st);
        hc.down(actions, da, na);
    });
    return rc == 0 ? VLA_OK : VLA_ERR_EXCEPTION;  // impact_capi.cpp:53-68
}

VLA_API int32_t vla_impact_predict_dev(void* h, const uint8_t* frames, const float* state, int32_t unnormalize,
                                       float* actions, void* stream) {
    if (!h || !frames || !state || !actions) return VLA_ERR_ARG;
    return guarded("vla_impact_predict_dev", [&] {
        impact_model(h)->predict_dev(frames, state, unnormalize != 0, actions, as_stream(stream));
    });
}

// impact_capi.cpp:70-87
VLA_API int32_t vla_impact_tokens(void* h, int32_t* ids, int32_t* compact, int32_t* mask, int32_t max_elems) {
    if (!h) return VLA_ERR_ARG;
    const ImpactModel& m = *impact_model(h);
    const int n = m.n_text();
    if (max_elems < n || m.token_ids().size() != (size_t)n) return VLA_ERR_ARG;
    for (int i = 0; i < n; i++) {
        if (ids) ids[i] = m.token_ids()[i];
        if (compact) compact[i] = m.compact_ids()[i];
        if (mask) mask[i] = m.token_mask()[i];
    }
    return n;
}

// impact_capi.cpp:89-101
VLA_API int32_t vla_impact_film(void* h, float* gamma, float* beta, int32_t max_elems) {
    if (!h) return VLA_ERR_ARG;
    const ImpactModel& m = *impact_model(h);
    const int n = (int)m.film_gamma().size();
    if (n == 0) return m.token_ids().empty() ? VLA_ERR_ARG : 0;
    if (max_elems < n) return VLA_ERR_ARG;
    if (gamma) std::memcpy(gamma, m.film_gamma().data(), sizeof(float) * (size_t)n);
    if (beta) std::memcpy(beta, m.film_beta().data(), sizeof(float) * (size_t)n);
    return n;
}

// ----------------------------------------- Diffusion Policy (model level) --
// The reference's Diffusion Policy entry points (include/vla_simd.h:245-280,
// src/models/diffusion/diffusion_capi.cpp), same names, signatures and status
// codes: the getters answer VLA_ERR_ARG for a null handle.

namespace {
DiffusionModel* dp_model(void* h) { return static_cast<DiffusionModel*>(h); }
}  // namespace

VLA_API void* vla_diffusion_load(const char* model_dir) {
    DiffusionModel* m = nullptr;
    const int32_t rc = guarded("vla_diffusion_load", [&] {
        VLA_REQUIRE(model_dir, "null model directory");
        m = new DiffusionModel(model_dir);
    });
    return rc == 0 ? m : nullptr;
}
VLA_API void vla_diffusion_free(void* h) { delete dp_model(h); }
VLA_API int32_t vla_diffusion_chunk(void* h) { return h ? dp_model(h)->chunk() : VLA_ERR_ARG; }
VLA_API int32_t vla_diffusion_horizon(void* h) { return h ? dp_model(h)->horizon() : VLA_ERR_ARG; }
VLA_API int32_t vla_diffusion_action_dim(void* h) { return h ? dp_model(h)->action_dim() : VLA_ERR_ARG; }
VLA_API int32_t vla_diffusion_state_dim(void* h) { return h ? dp_model(h)->state_dim() : VLA_ERR_ARG; }
VLA_API int32_t vla_diffusion_n_cams(void* h) { return h ? dp_model(h)->n_cams() : VLA_ERR_ARG; }
VLA_API int32_t vla_diffusion_n_obs_steps(void* h) { return h ? dp_model(h)->n_obs() : VLA_ERR_ARG; }
VLA_API int32_t vla_diffusion_img_h(void* h) { return h ? dp_model(h)->img_h() : VLA_ERR_ARG; }
VLA_API int32_t vla_diffusion_img_w(void* h) { return h ? dp_model(h)->img_w() : VLA_ERR_ARG; }
VLA_API int32_t vla_diffusion_num_steps(void* h) { return h ? dp_model(h)->num_steps() : VLA_ERR_ARG; }
VLA_API int32_t vla_diffusion_is_ddim(void* h) { return h ? (dp_model(h)->is_ddim() ? 1 : 0) : VLA_ERR_ARG; }
VLA_API int32_t vla_diffusion_int8_layers(void* h) { return h ? dp_model(h)->int8_layers() : 0; }
VLA_API int32_t vla_diffusion_int8_convs(void* h) { return h ? dp_model(h)->int8_convs() : 0; }
VLA_API int32_t vla_diffusion_graph_nodes(void* h) { return h ? dp_model(h)->graph_nodes() : 0; }

VLA_API int32_t vla_diffusion_predict(void* h, const uint8_t* frames, const float* state, int32_t unnormalize,
                                      float* actions, const float* noise) {
    if (!h || !frames || !state || !actions) return VLA_ERR_ARG;
    const int32_t rc = guarded("vla_diffusion_predict",
                               [&] { dp_model(h)->predict(frames, state, noise, unnormalize != 0, actions); });
    return rc == 0 ? VLA_OK : VLA_ERR_EXCEPTION;  // diffusion_capi.cpp:57-71
}

// -------------------------------------------------- SmolVLA (model level) --
// The reference's SmolVLA entry points (include/vla_simd.h:83-124,
// src/models/smolvla/smolvla_capi.cpp), same names and signatures.

namespace {
SmolvlaModel* smolvla_model(void* h) { return static_cast<SmolvlaModel*>(h); }
}  // namespace

VLA_API void* vla_smolvla_load(const char* model_dir, const char* tok_dir) {
    SmolvlaModel* m = nullptr;
    const int32_t rc = guarded("vla_smolvla_load", [&] {
        VLA_REQUIRE(model_dir && tok_dir, "null model or tokenizer directory");
        m = new SmolvlaModel(model_dir, tok_dir);
    });
    return rc == 0 ? m : nullptr;
}
VLA_API void vla_smolvla_free(void* h) { delete smolvla_model(h); }
VLA_API int32_t vla_smolvla_chunk(void* h) { return h ? smolvla_model(h)->chunk() : 0; }
VLA_API int32_t vla_smolvla_action_dim(void* h) { return h ? smolvla_model(h)->action_dim() : 0; }
VLA_API int32_t vla_smolvla_state_dim(void* h) { return h ? smolvla_model(h)->state_dim() : 0; }
VLA_API int32_t vla_smolvla_n_views(void* h) { return h ? smolvla_model(h)->n_views() : 0; }
VLA_API int32_t vla_smolvla_img_size(void* h) { return h ? smolvla_model(h)->img_size() : 0; }
VLA_API int32_t vla_smolvla_tok_maxlen(void* h) { return h ? smolvla_model(h)->tok_maxlen() : 0; }
VLA_API int32_t vla_smolvla_int8_layers(void* h) { return h ? smolvla_model(h)->int8_layers() : 0; }
VLA_API int32_t vla_smolvla_graph_nodes(void* h) { return h ? smolvla_model(h)->graph_nodes() : 0; }

VLA_API int32_t vla_smolvla_tokenize(void* h, const char* text, int32_t* ids, int32_t* mask) {
    if (!h || !text || !ids || !mask) return VLA_ERR_ARG;
    int32_t n = 0;
    const int32_t rc = guarded("vla_smolvla_tokenize", [&] { n = smolvla_model(h)->tokenize(text, ids, mask); });
    return rc == 0 ? n : VLA_ERR_EXCEPTION;
}

VLA_API int32_t vla_smolvla_predict_rtc(void* h, const uint8_t* frames, int32_t n_views, int32_t height,
                                        int32_t width, const int32_t* lang_tokens, const int32_t* lang_mask,
                                        int32_t n_lang, const float* state, const float* noise, uint64_t seed,
                                        float* actions, const float* prev, int32_t n_prev, const float* weights,
                                        float max_guidance) {
    if (!h || !frames || !lang_tokens || !lang_mask || !state || !actions) return VLA_ERR_ARG;
    return guarded("vla_smolvla_predict_rtc", [&] {
        smolvla_model(h)->predict(frames, n_views, height, width, lang_tokens, lang_mask, n_lang, state, noise, seed,
                                  actions, prev, n_prev, weights, max_guidance);
    });
}

VLA_API int32_t vla_smolvla_predict(void* h, const uint8_t* frames, int32_t n_views, int32_t height, int32_t width,
                                    const int32_t* lang_tokens, const int32_t* lang_mask, int32_t n_lang,
                                    const float* state, const float* noise, uint64_t seed, float* actions) {
    return vla_smolvla_predict_rtc(h, frames, n_views, height, width, lang_tokens, lang_mask, n_lang, state, noise,
                                   seed, actions, nullptr, 0, nullptr, 0.0f);
}

VLA_API int32_t vla_smolvla_preprocess(void* h, const uint8_t* frames, int32_t n_views, int32_t height,
                                       int32_t width, float* pixels) {
    if (!h || !frames || !pixels) return VLA_ERR_ARG;
    return guarded("vla_smolvla_preprocess",
                   [&] { smolvla_model(h)->preprocess(frames, n_views, height, width, pixels); });
}

// ------------------------------------------------------ the BPE tokenizer --
// SmolVLA's tokenizer on its own (host code, no device needed), for callers
// that tokenize away from a loaded model and for tests.

VLA_API void* vla_bpe_load(const char* tok_dir) {
    BpeTokenizer* t = nullptr;
    const int32_t rc = guarded("vla_bpe_load", [&] {
        VLA_REQUIRE(tok_dir, "null tokenizer directory");
        auto read = [&](const char* name) {
            const std::string path = std::string(tok_dir) + "/" + name;
            FILE* f = std::fopen(path.c_str(), "rb");
            VLA_REQUIRE(f, "cannot open " + path);
            std::string s;
            char buf[65536];
            size_t n;
            while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) s.append(buf, n);
            std::fclose(f);
            return s;
        };
        auto tok = std::make_unique<BpeTokenizer>();
        VLA_REQUIRE(tok->load(read("vocab.txt"), read("merges.txt")), "empty vocab.txt or merges.txt");
        t = tok.release();
    });
    return rc == 0 ? t : nullptr;
}
VLA_API void vla_bpe_free(void* h) { delete static_cast<BpeTokenizer*>(h); }
VLA_API int32_t vla_bpe_encode(void* h, const char* text, int32_t* ids, int32_t cap) {
    if (!h || !text || cap < 0 || (cap > 0 && !ids)) return VLA_ERR_ARG;
    int32_t n = 0;
    const int32_t rc = guarded("vla_bpe_encode", [&] {
        const std::vector<int32_t> v = static_cast<BpeTokenizer*>(h)->encode(text);
        n = (int32_t)v.size();
        for (int32_t i = 0; i < n && i < cap; i++) ids[i] = v[i];
    });
    return rc == 0 ? n : rc;
}

// ---------------------------------------------------- the T5 tokenizer --
// Octo's SentencePiece unigram tokenizer on its own (host code).

namespace {
std::string read_file_text(const std::string& path) {
    FILE* f = std::fopen(path.c_str(), "rb");
    VLA_REQUIRE(f, "cannot open " + path);
    std::string s;
    char buf[65536];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) s.append(buf, n);
    std::fclose(f);
    return s;
}
}  // namespace

VLA_API void* vla_unigram_load(const char* tok_dir) {
    UnigramTokenizer* t = nullptr;
    const int32_t rc = guarded("vla_unigram_load", [&] {
        VLA_REQUIRE(tok_dir, "null tokenizer directory");
        auto tok = std::make_unique<UnigramTokenizer>();
        VLA_REQUIRE(tok->load(read_file_text(std::string(tok_dir) + "/vocab.txt")), "vocab.txt has no pieces");
        t = tok.release();
    });
    return rc == 0 ? t : nullptr;
}
VLA_API void vla_unigram_free(void* h) { delete static_cast<UnigramTokenizer*>(h); }
VLA_API int32_t vla_unigram_encode(void* h, const char* text, int32_t max_len, int32_t* ids) {
    if (!h || !text || !ids || max_len < 1) return VLA_ERR_ARG;
    return guarded("vla_unigram_encode", [&] {
        const std::vector<int32_t> v = static_cast<UnigramTokenizer*>(h)->encode(text, max_len);
        for (int32_t i = 0; i < max_len; i++) ids[i] = v[i];
    });
}

// ----------------------------------------------------- Octo (model level) --
// The reference's Octo entry points (include/vla_simd.h:126-153,
// src/models/octo/octo_capi.cpp), same names and signatures.

namespace {
OctoModel* octo_model(void* h) { return static_cast<OctoModel*>(h); }
}  // namespace

VLA_API void* vla_octo_load(const char* model_dir, const char* tok_dir) {
    OctoModel* m = nullptr;
    const int32_t rc = guarded("vla_octo_load", [&] {
        VLA_REQUIRE(model_dir && tok_dir, "null model or tokenizer directory");
        m = new OctoModel(model_dir, tok_dir);
    });
    return rc == 0 ? m : nullptr;
}
VLA_API void vla_octo_free(void* h) { delete octo_model(h); }
VLA_API int32_t vla_octo_horizon(void* h) { return h ? octo_model(h)->horizon() : 0; }
VLA_API int32_t vla_octo_action_dim(void* h) { return h ? octo_model(h)->action_dim() : 0; }
VLA_API int32_t vla_octo_max_window(void* h) { return h ? octo_model(h)->max_window() : 0; }
VLA_API int32_t vla_octo_int8_layers(void* h) { return h ? octo_model(h)->int8_layers() : 0; }

VLA_API int32_t vla_octo_predict_ex(void* h, const uint8_t* primary, const uint8_t* wrist, int32_t wnd,
                                    const uint8_t* timestep_mask, const char* instruction, const float* noise,
                                    const float* z, uint64_t seed, int32_t unnormalize, float* actions) {
    if (!h || !primary || !timestep_mask || !instruction || !actions) return VLA_ERR_ARG;
    return guarded("vla_octo_predict_ex", [&] {
        octo_model(h)->predict(primary, wrist, wnd, timestep_mask, instruction, noise, z, seed, unnormalize != 0,
                               actions);
    });
}

VLA_API int32_t vla_octo_predict(void* h, const uint8_t* primary, const uint8_t* wrist, int32_t wnd,
                                 const uint8_t* timestep_mask, const char* instruction, uint64_t seed,
                                 int32_t unnormalize, float* actions) {
    return vla_octo_predict_ex(h, primary, wrist, wnd, timestep_mask, instruction, nullptr, nullptr, seed,
                               unnormalize, actions);
}

VLA_API int32_t vla_octo_lang(void* h, const char* instruction, float* out, int64_t n) {
    if (!h || !instruction || !out) return VLA_ERR_ARG;
    return guarded("vla_octo_lang", [&] {
        VLA_REQUIRE(n == octo_model(h)->lang_size(), "vla_octo_lang: n must be n_task * t5_dim");
        octo_model(h)->lang(instruction, out);
    });
}
