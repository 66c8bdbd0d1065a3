// model_act.cpp - the ACT transformer on the device (see models.h).
//
// Follows src/models/act/act_transformer.cpp: load() reads act.meta / act.bin
// in the order of :29-170 (the same float arena walk), build_tokens :212-250,
// encode :252-301, decode :303-356. What differs is only where values live and
// how launches are grouped, never a value:
//   - q and k of a self-attention read the same input (x + pos), so their
//     weights are row-concatenated into one int8 layer: one quantization of the
//     input (MhaQKV's shared_qk, src/nn/attention.cpp:40-59) and one GEMM;
//   - the wo and w2 residual adds (x[i] += resid[i], :273-277, :286-290) are the
//     GEMM epilogue's accumulate (x + v, the same single rounding);
//   - relu after w1 (:283) is the GEMM epilogue's activation;
//   - all cameras' tokens go through img_proj as one GEMM (quantization is per
//     row, so batching rows changes nothing).
#include "ckpt.h"
#include "models.h"

#include <cmath>

namespace vla {
namespace hip {

namespace {

// Float-arena cursor over a .bin (ArenaCursor, src/models/arena.h:68-80).
struct Cursor {
    const float* p;
    size_t n, off = 0;
    const float* take(size_t k) {
        if (k > n - off) throw ArgError("checkpoint .bin is shorter than its .meta says");
        const float* r = p + off;
        off += k;
        return r;
    }
};

// ActTransformer::sinusoid_pos_2d (act_transformer.cpp:189-210): the 2D
// sinusoidal camera embedding, the y half then the x half; float arithmetic
// and float libm, as the reference computes it on the host.
void sinusoid_pos_2d(int fh, int fw, int dim, float* out) {
    const int half = dim / 2;
    const float two_pi = 6.283185307179586f, eps = 1e-6f;
    std::vector<float> inv_freq(half);
    for (int c = 0; c < half; c++) inv_freq[c] = std::pow(10000.0f, (float)(2 * (c / 2)) / (float)half);
    for (int i = 0; i < fh; i++) {
        const float yr = (float)(i + 1) / ((float)fh + eps) * two_pi;
        for (int j = 0; j < fw; j++) {
            const float xr = (float)(j + 1) / ((float)fw + eps) * two_pi;
            float* o = out + (size_t)(i * fw + j) * dim;
            for (int c = 0; c < half; c++) {
                const float y = yr / inv_freq[c], x = xr / inv_freq[c];
                o[c] = (c & 1) ? std::cos(y) : std::sin(y);
                o[half + c] = (c & 1) ? std::cos(x) : std::sin(x);
            }
        }
    }
}

}  // namespace

ActTf::ActTf(const std::string& dir, int img_ch, int int8_mask, bool int8_state, const std::string& tag) {
    const CkptFiles files(dir);  // a converted directory or a vla.simd GGUF
    const std::string mf = tag + ".meta", bf = tag + ".bin";
    // act_transformer.cpp:31-52: each known key's value is read as `ss >> int`
    // (ln_eps as float) and the rest of its line must be blank; unknown keys
    // are skipped
    int& n_text = n_text_;
    for (const auto& kv : files.meta_lines(mf)) {
        const std::string& k = kv.first;
        int* dst = k == "dim" ? &d_ : k == "heads" ? &heads_ : k == "head_dim" ? &hd_ : k == "ff" ? &ff_
                 : k == "n_enc" ? &n_enc_ : k == "n_dec" ? &n_dec_ : k == "chunk" ? &chunk_
                 : k == "state_dim" ? &state_dim_ : k == "action_dim" ? &action_dim_ : k == "n_1d" ? &n_1d_
                 : k == "n_text" ? &n_text : nullptr;
        if (dst) *dst = meta_value_int(mf, k, kv.second);
        else if (k == "ln_eps") eps_ = meta_value_float(mf, k, kv.second);
    }
    img_ch_ = img_ch;
    VLA_REQUIRE(d_ > 0 && d_ % 4 == 0 && heads_ > 0 && hd_ > 0 && heads_ * hd_ == d_ && ff_ > 0 &&
                    chunk_ > 0 && state_dim_ > 0 && action_dim_ > 0 && img_ch > 0 && n_enc_ >= 1 &&
                    n_dec_ >= 1 && n_1d_ == 2 && n_text >= 0 && std::isfinite(eps_) && eps_ > 0,
                mf + ": invalid configuration (act_transformer.cpp:56-62 bounds)");

    const std::vector<char> raw = files.bytes(bf);
    VLA_REQUIRE(raw.size() % 4 == 0, bf + ": size is not a whole number of floats");
    Cursor take{reinterpret_cast<const float*>(raw.data()), raw.size() / 4};
    const int d = d_;
    auto lin = [&](DLinear& L, int N, int K, bool i8) {
        const float* w = take.take((size_t)N * K);
        const float* b = take.take(N);
        L.init(A_, w, b, N, K, i8);
        n_int8_ += i8;
    };
    struct Mha {
        const float *wq, *bq, *wk, *bk, *wv, *bv, *wo, *bo;
    };
    auto mha = [&]() {
        Mha h;
        h.wq = take.take((size_t)d * d); h.bq = take.take(d);
        h.wk = take.take((size_t)d * d); h.bk = take.take(d);
        h.wv = take.take((size_t)d * d); h.bv = take.take(d);
        h.wo = take.take((size_t)d * d); h.bo = take.take(d);
        return h;
    };
    auto vec = [&](size_t k) { return A_.upload(take.take(k), k); };

    lin(img_proj_, d, img_ch, int8_mask & 8);
    // Role::Generic, fp32 (:142-145) unless IMPACT's int8_state joins it to
    // the img_proj group (:127-130)
    lin(state_proj_, d, state_dim_, int8_state && (int8_mask & 8));
    latent_ = vec(d);
    pos1d_ = vec((size_t)n_1d_ * d);

    const bool ia = int8_mask & 1, i1 = int8_mask & 2, i2 = int8_mask & 4, idec = int8_mask & 16;
    enc_.resize(n_enc_);
    for (Enc& l : enc_) {
        const Mha h = mha();
        l.qk.init(A_, {{h.wq, h.bq, d}, {h.wk, h.bk, d}}, d, ia);
        l.v.init(A_, h.wv, h.bv, d, d, ia);
        l.o.init(A_, h.wo, h.bo, d, d, ia);
        n_int8_ += ia ? 4 : 0;
        l.n1s = vec(d);
        l.n1b = vec(d);
        lin(l.w1, ff_, d, i1);
        lin(l.w2, d, ff_, i2);
        l.n2s = vec(d);
        l.n2b = vec(d);
    }
    dec_.resize(n_dec_);
    for (Dec& l : dec_) {
        const Mha s = mha();
        l.sqk.init(A_, {{s.wq, s.bq, d}, {s.wk, s.bk, d}}, d, idec);
        l.sv.init(A_, s.wv, s.bv, d, d, idec);
        l.so.init(A_, s.wo, s.bo, d, d, idec);
        l.n1s = vec(d);
        l.n1b = vec(d);
        const Mha c = mha();
        l.cq.init(A_, c.wq, c.bq, d, d, idec);
        l.ck.init(A_, c.wk, c.bk, d, d, idec);
        l.cv.init(A_, c.wv, c.bv, d, d, idec);
        l.co.init(A_, c.wo, c.bo, d, d, idec);
        n_int8_ += idec ? 8 : 0;
        l.n2s = vec(d);
        l.n2b = vec(d);
        lin(l.w1, ff_, d, idec);
        lin(l.w2, d, ff_, idec);
        l.n3s = vec(d);
        l.n3b = vec(d);
    }
    dec_pos_ = vec((size_t)chunk_ * d);
    dec_ns_ = vec(d);
    dec_nb_ = vec(d);
    lin(head_, action_dim_, d, false);  // Role::Generic, fp32 (:142-145)
    VLA_REQUIRE(take.off == take.n, bf + ": size does not match " + mf);
    VLA_HIP_CHECK(hipStreamCreateWithFlags(&own_, hipStreamNonBlocking));
}

ActTf::~ActTf() {
    if (own_) (void)hipStreamDestroy(own_);
}

void ActTf::ensure(int n_cams, int fh, int fw, int nt) {
    if (n_cams == n_cams_ && fh == fh_ && fw == fw_ && nt == nt_) return;
    VLA_REQUIRE(n_cams > 0 && fh > 0 && fw > 0 && (long)n_cams * fh * fw < (1 << 20),
                "act: camera grid out of range");
    VLA_HIP_CHECK(hipDeviceSynchronize());
    S_.reset();
    auto S = std::make_unique<DeviceArena>();
    const int T = n_tokens(n_cams, fh, fw, nt), d = d_, C = chunk_;
    const int n_img = fh * fw;
    feats_ = S->alloc<float>((size_t)n_cams * n_img * img_ch_);
    state_ = S->alloc<float>(state_dim_);
    act_out_ = S->alloc<float>((size_t)C * action_dim_);
    // buffers the encoder (T rows) and the decoder (C rows) share take the larger
    const int R = T > C ? T : C;
    x_ = S->alloc<float>((size_t)T * d);
    xp_ = S->alloc<float>((size_t)R * d);
    qk_ = S->alloc<float>((size_t)R * 2 * d);
    v_ = S->alloc<float>((size_t)R * d);
    att_ = S->alloc<float>((size_t)R * d);
    ff_buf_ = S->alloc<float>((size_t)R * ff_);
    dx_ = S->alloc<float>((size_t)C * d);
    zero_ = S->alloc<float>((size_t)C * d);
    kpos_ = S->alloc<float>((size_t)T * d);
    ckb_ = S->alloc<float>((size_t)n_dec_ * T * d);
    cvb_ = S->alloc<float>((size_t)n_dec_ * T * d);
    dq_ = S->alloc<float>((size_t)C * d);
    text_ = nt ? S->alloc<float>((size_t)nt * d) : nullptr;
    // positions: [pos1d | camera embedding per camera | text positions, copied
    // in per call] (build_tokens :218-249)
    std::vector<float> pos((size_t)T * d), cam((size_t)n_img * d);
    sinusoid_pos_2d(fh, fw, d, cam.data());
    std::vector<float> p1((size_t)n_1d_ * d);
    VLA_HIP_CHECK(hipMemcpy(p1.data(), pos1d_, p1.size() * 4, hipMemcpyDeviceToHost));
    std::copy(p1.begin(), p1.end(), pos.begin());
    for (int c = 0; c < n_cams; c++)
        std::copy(cam.begin(), cam.end(), pos.begin() + ((size_t)n_1d_ + (size_t)c * n_img) * d);
    pos_ = S->upload(pos.data(), pos.size());
    // quantization scratch: the widest int8 input is ff (w2) over T rows
    int maxld = round_up(kpad4(ff_ > img_ch_ ? ff_ : img_ch_), 64);
    if (round_up(kpad4(d), 64) > maxld) maxld = round_up(kpad4(d), 64);
    ctx_.alloc(*S, R, maxld);
    S_ = std::move(S);
    n_cams_ = n_cams;
    fh_ = fh;
    fw_ = fw;
    nt_ = nt;
    T_ = T;
}

// VLA_HIP_ACT_HEAD=0 recomputes decoder layer 0's self-attention block on
// every forward (read per call; A/B runs and the bit-exactness test)
static bool head_hoist_on() {
    const char* e = std::getenv("VLA_HIP_ACT_HEAD");
    return !(e && e[0] == '0' && e[1] == '\0');
}

void ActTf::run(hipStream_t st, bool head_only) {
    Ctx c = ctx_;
    c.st = st;
    const int T = T_, d = d_, C = chunk_, n_img = fh_ * fw_;
    const float scale = 1.0f / std::sqrt((float)hd_);
    const MaskSpec none;

    // The row kernel that ends each block (and the token assembly) also
    // quantizes what the next block's projections read: x + pos for q | k
    // (slot 0) and x for v (slot 1), so no layer quantizes its own input.
    // row op over x (in place), quantizing x -> slot 1 and x + add -> slot 0 for
    // the consumers qk / v (fp32 consumers get xp_ / x_ rows instead)
    auto feed = [&](int op, float* x, int rows, const float* w, const float* b, const float* add,
                    const DLinear& qk, const DLinear& v, In& in_qk, In& in_v) {
        RowQArgs r;
        r.op = op;
        r.x = x;
        r.ldx = d;
        r.w = w;
        r.b = b;
        r.eps = eps_;
        r.rows = rows;
        r.H = d;
        r.out = op ? x : nullptr;
        r.ldo = d;
        r.add = add;
        r.ld_add = d;
        in_qk = In();
        in_v = In();
        in_v.f = x;
        in_v.ldf = d;
        if (v.int8()) {
            in_v.q = c.slot(1, v.ldq(), rows);
            in_v.quantized = true;
            r.q = in_v.q.q;
            r.ldq = in_v.q.ld;
            r.qs = in_v.q.s;
            r.q_panel = in_v.q.panel ? 1 : 0;
        }
        in_qk.f = xp_;
        in_qk.ldf = d;
        if (qk.int8()) {
            in_qk.q = c.slot(0, qk.ldq(), rows);  // same rows: same layout as q
            in_qk.quantized = true;
            r.q2 = in_qk.q.q;
            r.ldq2 = in_qk.q.ld;
            r.qs2 = in_qk.q.s;
            r.q_panel = in_qk.q.panel ? 1 : 0;
        } else {
            r.out2 = xp_;
            r.ldo2 = d;
        }
        rowq(r, st);
    };
    auto norm_for = [&](float* x, int rows, const float* w, const float* b, const DLinear& next) {
        RowQArgs r;
        r.op = 1;
        r.x = x;
        r.ldx = d;
        r.w = w;
        r.b = b;
        r.eps = eps_;
        r.rows = rows;
        r.H = d;
        return rowop_for(c, next, r, x, d, 0);  // in place, as layernorm(x, x)
    };

    In in_qk, in_v;
    // decoder layer 0's self-attention block and norm1 (decode, :303-325)
    // read only the zero queries, dec_pos and weights, so their outputs are
    // the same every forward: computed once (head_only) and copied in after
    const bool use_head = !head_only && head_done_ && head_hoist_on() && !probe_on();
    if (!head_only) {
        // build_tokens (:212-250): latent, state projection, camera tokens
        copy_f32(x_, latent_, d, st);
        linear(c, state_proj_, x_ + d, d, state_, state_dim_, 1);
        linear(c, img_proj_, x_ + (size_t)n_1d_ * d, d, feats_, img_ch_, n_cams_ * n_img);
        if (nt_ > 0) copy_f32(x_ + ((size_t)n_1d_ + (size_t)n_cams_ * n_img) * d, text_, (int64_t)nt_ * d, st);

        // encode (:252-301)
        feed(0, x_, T, nullptr, nullptr, pos_, enc_[0].qk, enc_[0].v, in_qk, in_v);
        for (size_t li = 0; li < enc_.size(); li++) {
            const Enc& l = enc_[li];
            linear_pair(c, l.qk, in_qk, qk_, 2 * d, l.v, in_v, v_, d, T);  // q | k from x + pos, v from x
            attend(st, att_, d, qk_, 2 * d, qk_ + d, 2 * d, v_, d, T, T, heads_, heads_, hd_, scale, none);
            linear(c, l.o, x_, d, att_, d, T, 0, 1);  // x += wo(att)
            const In h = norm_for(x_, T, l.n1s, l.n1b, l.w1);
            linear(c, l.w1, h, ff_buf_, ff_, T, 1);  // relu
            linear(c, l.w2, x_, d, ff_buf_, ff_, T, 0, 1);
            // LN2, then the next block's inputs (or, after the last, the memory the
            // decoder's cross-attention reads: keys from x + pos, values from x)
            const DLinear& nqk = li + 1 < enc_.size() ? enc_[li + 1].qk : dec_[0].ck;
            const DLinear& nv = li + 1 < enc_.size() ? enc_[li + 1].v : dec_[0].cv;
            feed(1, x_, T, l.n2s, l.n2b, pos_, nqk, nv, in_qk, in_v);
        }

        // decode (:303-356). The cross-attention keys and values depend only on the
        // encoder output, so each layer's are projected here, before the decoder.
        for (size_t li = 0; li < dec_.size(); li++) {
            const Dec& l = dec_[li];
            if (li > 0) feed(0, x_, T, nullptr, nullptr, pos_, l.ck, l.cv, in_qk, in_v);
            linear_pair(c, l.ck, in_qk, ckb_ + (size_t)li * T * d, d, l.cv, in_v, cvb_ + (size_t)li * T * d, d, T);
        }
    }  // !head_only

    if (!use_head) {
        copy_f32(dx_, zero_, (int64_t)C * d, st);  // queries start at zero
        feed(0, dx_, C, nullptr, nullptr, dec_pos_, dec_[0].sqk, dec_[0].sv, in_qk, in_v);
    }
    for (size_t li = 0; li < dec_.size(); li++) {
        const Dec& l = dec_[li];
        In in_q;
        in_q.f = xp_;
        in_q.ldf = d;
        if (li == 0 && use_head) {
            copy_f32(dx_, head_dx_, (int64_t)C * d, st);
            if (l.cq.int8()) {
                in_q.q = c.slot(0, l.cq.ldq(), C);  // the layout the slot gives these rows
                in_q.q.q = head_q_;
                in_q.q.s = head_qs_;
                in_q.quantized = true;
            } else {
                in_q.f = head_xp_;
            }
        } else {
            linear_pair(c, l.sqk, in_qk, qk_, 2 * d, l.sv, in_v, v_, d, C);
            attend(st, att_, d, qk_, 2 * d, qk_ + d, 2 * d, v_, d, C, C, heads_, heads_, hd_, scale, none);
            linear(c, l.so, dx_, d, att_, d, C, 0, 1);
            // LN1, then the cross query input dx + dec_pos
            RowQArgs r;
            r.op = 1;
            r.x = dx_;
            r.ldx = d;
            r.w = l.n1s;
            r.b = l.n1b;
            r.eps = eps_;
            r.rows = C;
            r.H = d;
            r.out = dx_;
            r.ldo = d;
            r.add = dec_pos_;
            r.ld_add = d;
            if (l.cq.int8()) {
                in_q.q = c.slot(0, l.cq.ldq(), C);
                in_q.quantized = true;
                r.q2 = in_q.q.q;
                r.ldq2 = in_q.q.ld;
                r.qs2 = in_q.q.s;
                r.q_panel = in_q.q.panel ? 1 : 0;
            } else {
                r.out2 = xp_;
                r.ldo2 = d;
            }
            rowq(r, st);
            if (head_only) return;
        }
        linear(c, l.cq, in_q, dq_, d, C);
        attend(st, att_, d, dq_, d, ckb_ + (size_t)li * T * d, d, cvb_ + (size_t)li * T * d, d, C, T,
               heads_, heads_, hd_, scale, none);
        linear(c, l.co, dx_, d, att_, d, C, 0, 1);
        const In h = norm_for(dx_, C, l.n2s, l.n2b, l.w1);
        linear(c, l.w1, h, ff_buf_, ff_, C, 1);
        linear(c, l.w2, dx_, d, ff_buf_, ff_, C, 0, 1);
        if (li + 1 < dec_.size())
            feed(1, dx_, C, l.n3s, l.n3b, dec_pos_, dec_[li + 1].sqk, dec_[li + 1].sv, in_qk, in_v);
        else
            launch_layernorm(dx_, dx_, l.n3s, l.n3b, C, d, eps_, st);
    }
    launch_layernorm(dx_, dx_, dec_ns_, dec_nb_, C, d, eps_, st);
    linear(c, head_, act_out_, action_dim_, dx_, d, C);
}

void ActTf::forward_text_dev(const float* feats, int n_cams, int fh, int fw, const float* state_norm,
                             const float* text, const float* text_pos, int n_text_real, float* actions_norm,
                             hipStream_t caller) {
    VLA_REQUIRE(feats && state_norm && actions_norm, "act: null buffer");
    // clamp_text (act_transformer.h:79): only real text tokens enter the sequence
    const int nt = n_text_real < 0 ? 0 : n_text_real > n_text_ ? n_text_ : n_text_real;
    VLA_REQUIRE(nt == 0 || (text && text_pos), "act: text tokens without their positions");
    ensure(n_cams, fh, fw, nt);
    if (!head_done_ && head_hoist_on() && !probe_on()) {
        // decoder layer 0's self-attention block, once per model, eagerly on
        // the caller's stream (before any graph is captured)
        const int C = chunk_, d = d_;
        const Dec& l = dec_[0];
        const QAct q = ctx_.slot(0, l.cq.ldq(), C);
        head_dx_ = A_.alloc<float>((size_t)C * d);
        if (l.cq.int8()) {
            head_q_bytes_ = q.panel ? (size_t)panel_rows(C) * q.ld : (size_t)C * q.ld;
            head_q_ = A_.alloc<int8_t>(head_q_bytes_);
            head_qs_ = A_.alloc<float>((size_t)C);
        } else {
            head_xp_ = A_.alloc<float>((size_t)C * d);
        }
        run(caller, true);
        copy_f32(head_dx_, dx_, (int64_t)C * d, caller);
        if (l.cq.int8()) {
            VLA_HIP_CHECK(hipMemcpyAsync(head_q_, q.q, head_q_bytes_, hipMemcpyDeviceToDevice, caller));
            copy_f32(head_qs_, q.s, C, caller);
        } else {
            copy_f32(head_xp_, xp_, (int64_t)C * d, caller);
        }
        VLA_HIP_CHECK(hipStreamSynchronize(caller));
        head_done_ = true;
    }
    copy_f32(feats_, feats, (int64_t)n_cams * fh * fw * img_ch_, caller);
    copy_f32(state_, state_norm, state_dim_, caller);
    if (nt > 0) {
        copy_f32(text_, text, (int64_t)nt * d_, caller);
        copy_f32(pos_ + ((size_t)n_1d_ + (size_t)n_cams * fh * fw) * d_, text_pos, (int64_t)nt * d_, caller);
    }
    const uint64_t key = ((uint64_t)nt << 50) | ((uint64_t)n_cams << 40) | ((uint64_t)fh << 20) | (uint64_t)fw;
    replay_.run(key, own_, caller, [this](hipStream_t st) { run(st); });
    copy_f32(actions_norm, act_out_, (int64_t)chunk_ * action_dim_, caller);
}

}  // namespace hip
}  // namespace vla
