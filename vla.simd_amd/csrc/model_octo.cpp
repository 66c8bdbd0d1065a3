// model_octo.cpp - the Octo block transformer on the device (see models.h).
//
// Follows src/models/octo/octo_transformer.cpp: load() reads octo.meta /
// octo.bin in the order of :17-99; forward :144-219 assembles the tokens, runs
// n_layers - 1 full pre-LN blocks (nn::EncoderLayer::forward,
// src/nn/encoder.cpp:26-77) and a readout-only last block
// (EncoderLayer::forward_last_row, encoder.cpp:79-113), then the final
// LayerNorm of the readout row. Value-preserving regroupings:
//   - the token assembly writes the positional rows first and adds each token
//     projection into them through the GEMM epilogue (pos + proj and proj + pos
//     are the same IEEE sum); the readout rows are the positional rows alone;
//   - q|k|v read one LayerNorm output, so they are one row-concatenated layer
//     behind one quantization (MhaQKV's shared_qk/shared_kv);
//   - the wo and w2 residual adds and gelu after w1 are GEMM epilogues;
//   - the additive [T, T] mask (:196-205) is a group table: a token's group is
//     (kind, timestep) and allow[gi][gj] = attends() && key not padded, which
//     blocks exactly the keys the mask sets to lowest().
#include "ckpt.h"
#include "models.h"

#include <cmath>

namespace vla {
namespace hip {

namespace {

struct Cursor {
    const float* p;
    size_t n, off = 0;
    const float* take(size_t k) {
        if (k > n - off) throw ArgError("octo.bin is shorter than octo.meta says");
        const float* r = p + off;
        off += k;
        return r;
    }
};

int meta_int(const std::map<std::string, double>& m, const char* k, int def) {
    return vla::hip::meta_int(m, "octo.meta", k, def);
}

// octo_transformer.cpp:103-109. Kinds: 0 task prefix (timestep -1), 1 primary,
// 2 wrist, 3 repeated task, 4 readout.
bool attends(int gi, int ti, int gj, int tj) {
    if (gi == 0) return gj == 0;
    if (gj == 0) return true;
    if (gj <= 3) return tj <= ti;
    return gi == 4 && gj == 4 && tj <= ti;
}

}  // namespace

OctoTf::OctoTf(const std::string& dir, int int8_mask) {
    const CkptFiles files(dir);  // a converted directory or a vla.simd GGUF
    const auto m = files.meta("octo.meta");
    d_ = meta_int(m, "d", d_);
    n_layers_ = meta_int(m, "n_layers", n_layers_);
    heads_ = meta_int(m, "heads", heads_);
    hd_ = meta_int(m, "head_dim", hd_);
    mlp_ = meta_int(m, "mlp", mlp_);
    max_h_ = meta_int(m, "max_horizon", max_h_);
    n_task_ = meta_int(m, "n_task", n_task_);
    tok_p_ = meta_int(m, "tok_primary", tok_p_);
    tok_w_ = meta_int(m, "tok_wrist", tok_w_);
    n_readout_ = meta_int(m, "n_readout", n_readout_);
    t5_dim_ = meta_int(m, "t5_dim", t5_dim_);
    stem_dim_ = meta_int(m, "stem_dim", stem_dim_);
    repeat_task_ = meta_int(m, "repeat_task", 1) != 0;
    if (m.count("ln_eps")) eps_ = (float)m.at("ln_eps");
    if (m.count("gelu_erf")) gelu_erf_ = m.at("gelu_erf") != 0;
    VLA_REQUIRE(d_ > 0 && heads_ > 0 && hd_ > 0 && heads_ * hd_ == d_ && mlp_ > 0 && n_task_ > 0 &&
                    t5_dim_ > 0 && stem_dim_ > 0 && max_h_ > 0 && tok_p_ > 0 && tok_w_ > 0 &&
                    n_readout_ > 0 && n_layers_ >= 1 && std::isfinite(eps_) && eps_ > 0,
                "octo.meta: invalid configuration (octo_transformer.cpp:40-48 bounds)");

    const std::vector<char> raw = files.bytes("octo.bin");
    VLA_REQUIRE(raw.size() % 4 == 0, "octo.bin: size is not a whole number of floats");
    Cursor take{reinterpret_cast<const float*>(raw.data()), raw.size() / 4};
    const int D = d_;
    auto lin = [&](DLinear& L, int N, int K, bool i8) {
        const float* w = take.take((size_t)N * K);
        const float* b = take.take(N);
        L.init(A_, w, b, N, K, i8);
        n_int8_ += i8;
    };
    auto vec = [&](size_t k) { return A_.upload(take.take(k), k); };

    const bool ip = int8_mask & 8, ia = int8_mask & 1, i1 = int8_mask & 2, i2 = int8_mask & 4;
    lin(proj_task_, D, t5_dim_, ip);
    lin(proj_prim_, D, stem_dim_, ip);
    lin(proj_wrist_, D, stem_dim_, ip);
    pos_task_ = vec((size_t)n_task_ * D);
    pos_prim_ = vec((size_t)max_h_ * tok_p_ * D);
    pos_wrist_ = vec((size_t)max_h_ * tok_w_ * D);
    pos_readout_ = vec((size_t)max_h_ * n_readout_ * D);
    layers_.resize(n_layers_);
    for (Layer& L : layers_) {
        L.ln1s = vec(D);
        L.ln1b = vec(D);
        const float* wq = take.take((size_t)D * D);
        const float* bq = take.take(D);
        const float* wk = take.take((size_t)D * D);
        const float* bk = take.take(D);
        const float* wv = take.take((size_t)D * D);
        const float* bv = take.take(D);
        L.qkv.init(A_, {{wq, bq, D}, {wk, bk, D}, {wv, bv, D}}, D, ia);
        lin(L.o, D, D, ia);
        n_int8_ += ia ? 3 : 0;
        L.ln2s = vec(D);
        L.ln2b = vec(D);
        lin(L.w1, mlp_, D, i1);
        lin(L.w2, D, mlp_, i2);
    }
    final_s_ = vec(D);
    final_b_ = vec(D);
    VLA_REQUIRE(take.off == take.n, "octo.bin: size does not match octo.meta");
    VLA_HIP_CHECK(hipStreamCreateWithFlags(&own_, hipStreamNonBlocking));
}

OctoTf::~OctoTf() {
    if (own_) (void)hipStreamDestroy(own_);
}

void OctoTf::ensure(int wnd, const uint8_t* tmask, bool wrist) {
    VLA_REQUIRE(wnd >= 1 && wnd <= max_h_, "octo: window must be in [1, max_horizon]");
    VLA_REQUIRE(1 + 4 * wnd <= 256, "octo: window too long for the group mask");
    // the token layout and the mask tables depend on exactly these
    std::vector<uint8_t> layout(2 + wnd);
    layout[0] = (uint8_t)wnd;
    layout[1] = wrist ? 1 : 0;
    for (int t = 0; t < wnd; t++) layout[2 + t] = tmask[t] ? 1 : 0;
    if (S_ && layout == layout_) return;
    VLA_HIP_CHECK(hipDeviceSynchronize());
    S_.reset();
    auto S = std::make_unique<DeviceArena>();
    const int D = d_, per = per_step(), total = total_tokens(wnd);
    t5_ = S->alloc<float>((size_t)n_task_ * t5_dim_);
    sp_ = S->alloc<float>((size_t)wnd * tok_p_ * stem_dim_);
    sw_ = S->alloc<float>((size_t)wnd * tok_w_ * stem_dim_);
    out_ = S->alloc<float>(D);
    x_ = S->alloc<float>((size_t)total * D);
    P_ = S->alloc<float>((size_t)total * D);
    h_ = S->alloc<float>((size_t)total * D);
    qkv_ = S->alloc<float>((size_t)total * 3 * D);
    att_ = S->alloc<float>((size_t)total * D);
    ff_buf_ = S->alloc<float>((size_t)total * mlp_);

    // positional rows (forward :155-185): task rows and their per-step copies
    // get pos_task, observation rows their timestep's table, readouts
    // pos_readout; wrist rows stay zero without a wrist stem
    auto d2d = [&](float* dst, const float* src, size_t n) {
        VLA_HIP_CHECK(hipMemcpy(dst, src, n * 4, hipMemcpyDeviceToDevice));
    };
    d2d(P_, pos_task_, (size_t)n_task_ * D);
    for (int t = 0; t < wnd; t++) {
        float* row = P_ + ((size_t)n_task_ + (size_t)t * per) * D;
        d2d(row, pos_prim_ + (size_t)t * tok_p_ * D, (size_t)tok_p_ * D);
        row += (size_t)tok_p_ * D;
        if (wrist) d2d(row, pos_wrist_ + (size_t)t * tok_w_ * D, (size_t)tok_w_ * D);
        row += (size_t)tok_w_ * D;
        if (repeat_task_) {
            d2d(row, pos_task_, (size_t)n_task_ * D);
            row += (size_t)n_task_ * D;
        }
        d2d(row, pos_readout_ + (size_t)t * n_readout_ * D, (size_t)n_readout_ * D);
    }

    // group table (build_mask :111-142)
    const int G = 1 + 4 * wnd;
    std::vector<uint8_t> qg(total), allow((size_t)G * G);
    std::vector<int> gk(G), gt(G), gpad(G);
    gk[0] = 0;
    gt[0] = -1;
    gpad[0] = 1;
    for (int t = 0; t < wnd; t++)
        for (int k = 1; k <= 4; k++) {
            const int g = 1 + 4 * t + (k - 1);
            gk[g] = k;
            gt[g] = t;
            gpad[g] = k == 1 ? tmask[t] != 0 : k == 2 ? (wrist && tmask[t] != 0) : 1;
        }
    for (int i = 0; i < n_task_; i++) qg[i] = 0;
    for (int t = 0; t < wnd; t++) {
        int idx = n_task_ + t * per;
        for (int i = 0; i < tok_p_; i++) qg[idx++] = (uint8_t)(1 + 4 * t);
        for (int i = 0; i < tok_w_; i++) qg[idx++] = (uint8_t)(2 + 4 * t);
        if (repeat_task_)
            for (int i = 0; i < n_task_; i++) qg[idx++] = (uint8_t)(3 + 4 * t);
        for (int i = 0; i < n_readout_; i++) qg[idx++] = (uint8_t)(4 + 4 * t);
    }
    for (int a = 0; a < G; a++)
        for (int b = 0; b < G; b++) allow[(size_t)a * G + b] = attends(gk[a], gt[a], gk[b], gt[b]) && gpad[b];
    qg_ = S->upload(qg.data(), qg.size());
    allow_ = S->upload(allow.data(), allow.size());
    n_groups_ = G;

    int maxld = round_up(kpad4(mlp_), 64);
    for (int k : {D, t5_dim_, stem_dim_})
        if (round_up(kpad4(k), 64) > maxld) maxld = round_up(kpad4(k), 64);
    ctx_.alloc(*S, total, maxld);
    S_ = std::move(S);
    layout_ = std::move(layout);
    key_++;  // a new layout: the captured graph is rebuilt
    wnd_ = wnd;
    total_ = total;
    wrist_ = wrist;
}

void OctoTf::run(hipStream_t st) {
    Ctx c = ctx_;
    c.st = st;
    const int D = d_, T = total_, per = per_step(), wnd = wnd_;
    const float scale = 1.0f / std::sqrt((float)hd_);
    MaskSpec mask;
    mask.kind = 3;
    mask.n_groups = n_groups_;
    mask.qg = qg_;
    mask.kg = qg_;
    mask.allow = allow_;
    const int gelu = gelu_erf_ ? 3 : 2;

    // token assembly (:155-185)
    copy_f32(x_, P_, (int64_t)T * D, st);
    linear(c, proj_task_, x_, D, t5_, t5_dim_, n_task_, 0, 1);
    for (int t = 0; t < wnd; t++) {
        float* row = x_ + ((size_t)n_task_ + (size_t)t * per) * D;
        linear(c, proj_prim_, row, D, sp_ + (size_t)t * tok_p_ * stem_dim_, stem_dim_, tok_p_, 0, 1);
        row += (size_t)tok_p_ * D;
        if (wrist_) linear(c, proj_wrist_, row, D, sw_ + (size_t)t * tok_w_ * stem_dim_, stem_dim_, tok_w_, 0, 1);
        row += (size_t)tok_w_ * D;
        if (repeat_task_) linear(c, proj_task_, row, D, t5_, t5_dim_, n_task_, 0, 1);
    }

    // LayerNorm rows of x feeding layer L: quantized in the same kernel when L
    // is int8 (h_ gets the fp32 rows only when L is fp32)
    auto ln_for = [&](const float* x, int rows, const float* w, const float* b, const DLinear& L) {
        RowQArgs r;
        r.op = 1;
        r.x = x;
        r.ldx = D;
        r.w = w;
        r.b = b;
        r.eps = eps_;
        r.rows = rows;
        r.H = D;
        return rowop_for(c, L, r, L.int8() ? nullptr : h_, D, 0);
    };

    // blocks 0 .. n-2 (EncoderLayer::forward)
    for (int li = 0; li + 1 < n_layers_; li++) {
        const Layer& L = layers_[li];
        const In h1 = ln_for(x_, T, L.ln1s, L.ln1b, L.qkv);
        linear(c, L.qkv, h1, qkv_, 3 * D, T);
        attend(st, att_, D, qkv_, 3 * D, qkv_ + D, 3 * D, qkv_ + 2 * D, 3 * D, T, T, heads_, heads_, hd_,
               scale, mask);
        linear(c, L.o, x_, D, att_, D, T, 0, 1);
        const In h2 = ln_for(x_, T, L.ln2s, L.ln2b, L.w1);
        linear(c, L.w1, h2, ff_buf_, mlp_, T, gelu);
        linear(c, L.w2, x_, D, ff_buf_, mlp_, T, 0, 1);
    }

    // last block, readout row only (forward_last_row): K/V over every token
    const Layer& L = layers_.back();
    const int ro = readout_index(wnd);
    float* xr = x_ + (size_t)ro * D;
    const In h1 = ln_for(x_, T, L.ln1s, L.ln1b, L.qkv);
    linear(c, L.qkv, h1, qkv_ + D, 3 * D, T, 0, 0, D, 3 * D);  // k | v, every row
    In hr = h1;                                                   // q of the readout row
    if (hr.quantized) {
        VLA_REQUIRE(!hr.q.panel, "octo: the readout row needs row-major quantized rows");
        hr.q.q += (size_t)ro * hr.q.ld;
        hr.q.s += ro;
    }
    if (hr.f) hr.f += (size_t)ro * D;
    linear(c, L.qkv, hr, qkv_ + (size_t)ro * 3 * D, 3 * D, 1, 0, 0, 0, D);
    MaskSpec mr = mask;
    mr.qg = qg_ + ro;
    attend(st, att_, D, qkv_ + (size_t)ro * 3 * D, 3 * D, qkv_ + D, 3 * D, qkv_ + 2 * D, 3 * D, 1, T,
           heads_, heads_, hd_, scale, mr);
    linear(c, L.o, xr, D, att_, D, 1, 0, 1);
    const In h2 = ln_for(xr, 1, L.ln2s, L.ln2b, L.w1);
    linear(c, L.w1, h2, ff_buf_, mlp_, 1, gelu);
    linear(c, L.w2, xr, D, ff_buf_, mlp_, 1, 0, 1);
    launch_layernorm(out_, xr, final_s_, final_b_, 1, D, eps_, st);
}

void OctoTf::forward_dev(const float* t5, const float* stem_p, const float* stem_w, int wnd,
                         const uint8_t* timestep_mask, float* out, hipStream_t caller) {
    VLA_REQUIRE(t5 && stem_p && timestep_mask && out, "octo: null buffer");
    ensure(wnd, timestep_mask, stem_w != nullptr);
    copy_f32(t5_, t5, (int64_t)n_task_ * t5_dim_, caller);
    copy_f32(sp_, stem_p, (int64_t)wnd * tok_p_ * stem_dim_, caller);
    if (stem_w) copy_f32(sw_, stem_w, (int64_t)wnd * tok_w_ * stem_dim_, caller);
    replay_.run(key_, own_, caller, [this](hipStream_t st) { run(st); });
    copy_f32(out, out_, d_, caller);
}

}  // namespace hip
}  // namespace vla
