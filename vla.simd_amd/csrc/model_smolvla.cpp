// model_smolvla.cpp - the SmolVLA action chunk on the device (see models.h).
//
// Follows the reference's chunk after the vision tower and the embedding
// lookup: smolvla_model.cpp:252-285 (prefix-LM mask, positions, denoise mask),
// SmollmVlm::prefix_forward (src/models/smolvla/smollm2_lm.cpp:85-132) and
// ActionExpert::denoise / denoise_step (action_expert.cpp:237-395), with the
// weights of vlm.meta/vlm.bin (smollm2_lm.cpp:17-83: fp32 norms, then bf16
// matrices) and aex.meta/aex.bin (action_expert.cpp:60-172, fp32).
//
// Layout: each text layer L owns one buffer [n_prefix + chunk, QF + 2 KV]
// holding q | k | v per row. The tower's concatenated q|k|v GEMM fills the
// prefix rows (post-RoPE K and raw V are the reference's VlmKV cache); an
// expert self-attention layer writes its suffix q|k|v into the rows after
// them, so the prefix/suffix K/V concat of denoise_step (:321-330) is already
// in place and attention reads K and V over all n_prefix + chunk rows.
// Value-preserving regroupings otherwise as in the other graphs: shared
// quantization behind concatenated q|k|v and gate|up layers, residual adds as
// GEMM epilogues, one RoPE launch over the q and k heads when they share
// positions, the Euler update x += dt * v_t as the action_out_proj epilogue
// fmaf(dt, v, x).
#include "ckpt.h"
#include "models.h"

#include <algorithm>
#include <cstdint>
#include <cmath>
#include <limits>

namespace vla {
namespace hip {

namespace {

int meta_int(const std::map<std::string, double>& m, const char* k, int def) {
    return vla::hip::meta_int(m, "smolvla meta", k, def);
}

double meta_f(const std::map<std::string, double>& m, const char* k, double def) {
    auto it = m.find(k);
    return it == m.end() ? def : it->second;
}

}  // namespace

SmolvlaTf::SmolvlaTf(const std::string& dir, int int8_mask) {
    const CkptFiles files(dir);  // a converted directory or a vla.simd GGUF
    // ---- text tower (smollm2_lm.cpp:17-83)
    const auto vm = files.meta("vlm.meta");
    H_ = meta_int(vm, "hidden", H_);
    nq_ = meta_int(vm, "n_q", nq_);
    nkv_ = meta_int(vm, "n_kv", nkv_);
    hd_ = meta_int(vm, "head_dim", hd_);
    F_ = meta_int(vm, "ffn", F_);
    eps_ = (float)meta_f(vm, "eps", eps_);
    rope_base_ = (float)meta_f(vm, "rope_base", rope_base_);
    NL_ = meta_int(vm, "n_layers", NL_);
    VLA_REQUIRE(nq_ > 0 && nkv_ > 0 && nq_ % nkv_ == 0 && hd_ > 0 && hd_ % 2 == 0 && nq_ * hd_ == H_ &&
                    F_ > 0 && NL_ >= 1 && eps_ > 0 && rope_base_ > 0,
                "vlm.meta: invalid configuration (smollm2_lm.cpp:34-39 bounds)");
    const int QF = nq_ * hd_, KV = nkv_ * hd_;
    const bool ilm = int8_mask & 16, iex = int8_mask & 32;
    {
        const std::vector<char> raw = files.bytes("vlm.bin");
        const size_t fcount = (size_t)2 * H_ * NL_ + H_;
        const size_t per = (size_t)QF * H_ + (size_t)KV * H_ * 2 + (size_t)H_ * QF + (size_t)F_ * H_ * 2 +
                           (size_t)H_ * F_;
        VLA_REQUIRE(raw.size() == fcount * 4 + per * NL_ * 2, "vlm.bin: size does not match vlm.meta");
        const float* fn = reinterpret_cast<const float*>(raw.data());
        const uint16_t* wb = reinterpret_cast<const uint16_t*>(raw.data() + fcount * 4);
        vlm_.resize(NL_);
        for (int L = 0; L < NL_; L++) {
            vlm_[L].ln_in = A_.upload(fn + (size_t)2 * H_ * L, H_);
            vlm_[L].ln_post = A_.upload(fn + (size_t)2 * H_ * L + H_, H_);
        }
        std::vector<float> tmp;
        auto bf = [&](size_t n) {  // next n bf16 weights as fp32 (Linear::init_int8's rebuild)
            tmp.resize(n);
            for (size_t i = 0; i < n; i++) tmp[i] = bf16_to_f32(wb[i]);
            wb += n;
            return tmp;
        };
        for (int L = 0; L < NL_; L++) {
            VlmLayer& w = vlm_[L];
            const std::vector<float> q = bf((size_t)QF * H_), k = bf((size_t)KV * H_), v = bf((size_t)KV * H_);
            w.qkv.init(A_, {{q.data(), nullptr, QF}, {k.data(), nullptr, KV}, {v.data(), nullptr, KV}}, H_, ilm);
            const std::vector<float> o = bf((size_t)H_ * QF);
            w.o.init(A_, o.data(), nullptr, H_, QF, ilm);
            const std::vector<float> g = bf((size_t)F_ * H_), u = bf((size_t)F_ * H_);
            w.gu.init(A_, {{g.data(), nullptr, F_}, {u.data(), nullptr, F_}}, H_, ilm);
            const std::vector<float> dn = bf((size_t)H_ * F_);
            w.down.init(A_, dn.data(), nullptr, H_, F_, ilm);
            n_int8_ += ilm ? 7 : 0;
        }
    }

    // ---- action expert (action_expert.cpp:60-172)
    const auto am = files.meta("aex.meta");
    EH_ = meta_int(am, "expert_h", EH_);
    EF_ = meta_int(am, "expert_ffn", EF_);
    enq_ = meta_int(am, "n_q", enq_);
    enkv_ = meta_int(am, "n_kv", enkv_);
    ehd_ = meta_int(am, "head_dim", ehd_);
    eeps_ = (float)meta_f(am, "eps", eeps_);
    erope_ = (float)meta_f(am, "rope_base", erope_);
    ENL_ = meta_int(am, "n_layers", ENL_);
    san_ = meta_int(am, "self_attn_every_n", san_);
    C_ = meta_int(am, "chunk", C_);
    steps_ = meta_int(am, "num_steps", steps_);
    mad_ = meta_int(am, "max_action_dim", mad_);
    min_period_ = meta_f(am, "min_period", min_period_);
    max_period_ = meta_f(am, "max_period", max_period_);
    const int EQF = enq_ * ehd_, EKV = enkv_ * ehd_;
    VLA_REQUIRE(enq_ > 0 && enkv_ > 0 && enq_ % enkv_ == 0 && ehd_ % 2 == 0 && EH_ % 2 == 0 && EF_ > 0 &&
                    ENL_ >= 1 && C_ > 0 && steps_ >= 1 && mad_ > 0 && san_ >= 0 && eeps_ > 0 &&
                    erope_ > 0 && min_period_ > 0 && max_period_ > min_period_,
                "aex.meta: invalid configuration (action_expert.cpp:93-104 bounds)");
    // smolvla_model.cpp:81-83: the expert shares the tower's K/V width and reads
    // one tower layer per expert layer; the suffix q|k|v reuse the tower's layout
    VLA_REQUIRE(EKV == KV && ENL_ <= NL_ && ehd_ == hd_ && enkv_ == nkv_ && EQF == QF,
                "smolvla: expert and text tower disagree on heads / layers");
    {
        const std::vector<char> raw = files.bytes("aex.bin");
        VLA_REQUIRE(raw.size() % 4 == 0, "aex.bin: size is not a whole number of floats");
        const float* p = reinterpret_cast<const float*>(raw.data());
        const size_t n = raw.size() / 4;
        size_t off = 0;
        auto take = [&](size_t k) {
            if (k > n - off) throw ArgError("aex.bin is shorter than aex.meta says");
            const float* r = p + off;
            off += k;
            return r;
        };
        exp_.resize(ENL_);
        for (int L = 0; L < ENL_; L++) {
            ExpLayer& w = exp_[L];
            w.self = san_ > 0 && L % san_ == 0;
            const int kk = w.self ? EH_ : KV;
            w.ln_in = A_.upload(take(EH_), EH_);
            const float* q = take((size_t)EQF * EH_);
            const float* k = take((size_t)EKV * kk);
            const float* v = take((size_t)EKV * kk);
            if (w.self) {
                w.q_or_qkv.init(A_, {{q, nullptr, EQF}, {k, nullptr, EKV}, {v, nullptr, EKV}}, EH_, iex);
            } else {
                w.q_or_qkv.init(A_, q, nullptr, EQF, EH_, iex);
                w.k.init(A_, k, nullptr, EKV, kk, iex);
                w.v.init(A_, v, nullptr, EKV, kk, iex);
            }
            w.o.init(A_, take((size_t)EH_ * EQF), nullptr, EH_, EQF, iex);
            w.ln_post = A_.upload(take(EH_), EH_);
            const float* g = take((size_t)EF_ * EH_);
            const float* u = take((size_t)EF_ * EH_);
            w.gu.init(A_, {{g, nullptr, EF_}, {u, nullptr, EF_}}, EH_, iex);
            w.down.init(A_, take((size_t)EH_ * EF_), nullptr, EH_, EF_, iex);
            n_int8_ += iex ? 7 : 0;
        }
        out_norm_ = A_.upload(take(EH_), EH_);
        // flow-matching projections stay fp32 (smolvla_model.cpp:41-43)
        const float* w = take((size_t)EH_ * mad_);
        ain_.init(A_, w, take(EH_), EH_, mad_, false);
        w = take((size_t)EH_ * 2 * EH_);
        at1_.init(A_, w, take(EH_), EH_, 2 * EH_, false);
        w = take((size_t)EH_ * EH_);
        at2_.init(A_, w, take(EH_), EH_, EH_, false);
        w = take((size_t)mad_ * EH_);
        aout_.init(A_, w, take(mad_), mad_, EH_, false);
        VLA_REQUIRE(off == n, "aex.bin: size does not match aex.meta");
    }
    QKVW_ = QF + 2 * KV;
    VLA_HIP_CHECK(hipStreamCreateWithFlags(&own_, hipStreamNonBlocking));
}

SmolvlaTf::~SmolvlaTf() {
    if (own_) (void)hipStreamDestroy(own_);
}

void SmolvlaTf::ensure(const int32_t* pad, int np) {
    VLA_REQUIRE(np >= 2 && np <= 65536 - C_, "smolvla: prefix length out of range");
    VLA_REQUIRE(pad[np - 1] != 0, "smolvla: the last prefix token (state) must be real");
    // As in the reference (smolvla_model.cpp:224-246), a pad entry is a truth
    // value in the masks (nonzero = real) and its raw value is summed into the
    // positions, so any int32 is taken; the running sums must stay within
    // int32 (where the reference's int sum would overflow).
    {
        int64_t cum = 0;
        for (int j = 0; j < np; j++) {
            cum += pad[j];
            VLA_REQUIRE(cum - 1 >= INT32_MIN && cum + C_ <= INT32_MAX, "smolvla: pad sums overflow the positions");
        }
    }
    // the masks and positions depend on the whole pad vector
    std::vector<int32_t> padv(pad, pad + np);
    if (S_ && padv == pad_) return;
    VLA_HIP_CHECK(hipDeviceSynchronize());
    S_.reset();
    auto S = std::make_unique<DeviceArena>();
    const int QF = nq_ * hd_, KV = nkv_ * hd_, C = C_, SK = np + C, EH = EH_;
    prefix_in_ = S->alloc<float>((size_t)np * H_);
    noise_in_ = S->alloc<float>((size_t)C * mad_);
    act_out_ = S->alloc<float>((size_t)C * mad_);
    h_ = S->alloc<float>((size_t)np * H_);
    xn_ = S->alloc<float>((size_t)np * H_);
    // buffers the tower (np rows) and the expert (C rows) share take the larger
    const int R = np > C ? np : C;
    att_ = S->alloc<float>((size_t)R * QF);
    const int FW = F_ > EF_ ? F_ : EF_;
    gu_raw_ = S->alloc<float>((size_t)R * 2 * FW);
    gu_ = S->alloc<float>((size_t)R * FW);
    eh_ = S->alloc<float>((size_t)C * EH);
    ehn_ = S->alloc<float>((size_t)C * EH);
    eq_ = S->alloc<float>((size_t)C * QF);
    mlp1_ = S->alloc<float>((size_t)C * EH);
    x_ = S->alloc<float>((size_t)C * mad_);
    hf_ = S->alloc<float>((size_t)C * EH);
    v_ = S->alloc<float>((size_t)C * mad_);
    guide_ = S->alloc<float>((size_t)C * mad_);
    gweights_ = S->alloc<float>(C);
    gw_ = S->alloc<float>(steps_);
    qkv_.assign(NL_, nullptr);
    for (int L = 0; L < NL_; L++) qkv_[L] = S->alloc<float>((size_t)SK * QKVW_);
    ck_.assign(ENL_, nullptr);
    cv_.assign(ENL_, nullptr);
    for (int L = 0; L < ENL_; L++)
        if (!exp_[L].self) {
            ck_[L] = S->alloc<float>((size_t)np * KV);
            cv_[L] = S->alloc<float>((size_t)np * KV);
        }

    // prefix-LM mask and positions (smolvla_model.cpp:252-264): a token's group
    // is 2 * att + pad (att = 1 only for the state token, the last one); key j is
    // visible to query i iff att(j) <= att(i) and both are real
    std::vector<uint8_t> grp(np), allow(16, 0);
    for (int j = 0; j < np; j++) grp[j] = (uint8_t)(2 * (j == np - 1 ? 1 : 0) + (pad[j] ? 1 : 0));
    for (int gi = 0; gi < 4; gi++)
        for (int gj = 0; gj < 4; gj++)
            allow[gi * 4 + gj] = (gj >> 1) <= (gi >> 1) && (gi & 1) && (gj & 1);
    pgroup_ = S->upload(grp.data(), grp.size());
    pallow_ = S->upload(allow.data(), allow.size());
    std::vector<int32_t> pos(np), pos_full(C), pos_reb(C);
    int32_t cum = 0;  // in range: checked above
    for (int j = 0; j < np; j++) {
        cum += pad[j];
        pos[j] = cum - 1;
    }
    // denoise mask and positions (:266-275; rebased :248-252 of action_expert.cpp)
    for (int i = 0; i < C; i++) {
        pos_full[i] = cum + i;
        pos_reb[i] = i;
    }
    // the positions are fixed per prefix layout, so the RoPE tables are built once
    const std::vector<double> tp = rope_cos_sin(pos.data(), np, hd_, rope_base_);
    const std::vector<double> tf = rope_cos_sin(pos_full.data(), C, ehd_, erope_);
    const std::vector<double> tr = rope_cos_sin(pos_reb.data(), C, ehd_, erope_);
    rope_p_ = S->upload(tp.data(), tp.size());
    rope_full_ = S->upload(tf.data(), tf.size());
    rope_reb_ = S->upload(tr.data(), tr.size());
    bool all_real = true;
    for (int j = 0; j < np; j++) all_real = all_real && pad[j] != 0;
    dcausal_ = all_real;
    cnone_ = all_real;
    if (!all_real) {
        const float NEG = std::numeric_limits<float>::lowest();
        std::vector<float> dm((size_t)C * SK), cm((size_t)C * np);
        for (int i = 0; i < C; i++) {
            for (int j = 0; j < np; j++) dm[(size_t)i * SK + j] = cm[(size_t)i * np + j] = pad[j] ? 0.0f : NEG;
            for (int j = 0; j < C; j++) dm[(size_t)i * SK + np + j] = j <= i ? 0.0f : NEG;
        }
        dmask_ = S->upload(dm.data(), dm.size());
        cmask_ = S->upload(cm.data(), cm.size());
    }

    // per-step action_time buffers: the right half is the step's sinusoidal
    // time embedding (embed_suffix :186-203, double math), written once here
    at_.assign(steps_, nullptr);
    const int half = EH / 2;
    std::vector<float> at((size_t)C * 2 * EH, 0.0f), te(EH);
    for (int s = 0; s < steps_; s++) {
        const double td = 1.0 + s * (-1.0 / steps_);
        const float time = (float)td;
        for (int i = 0; i < half; i++) {
            const double frac = half == 1 ? 0.0 : (double)i / (double)(half - 1);
            const double period = min_period_ * std::pow(max_period_ / min_period_, frac);
            const double a = (2.0 * M_PI / period) * (double)time;
            te[i] = (float)std::sin(a);
            te[half + i] = (float)std::cos(a);
        }
        for (int t = 0; t < C; t++) std::copy(te.begin(), te.end(), at.begin() + (size_t)t * 2 * EH + EH);
        at_[s] = S->upload(at.data(), at.size());
    }

    int maxld = 0;
    for (int k : {H_, QF, F_, EH, EF_, KV, 2 * EH})
        if (round_up(kpad4(k), 64) > maxld) maxld = round_up(kpad4(k), 64);
    ctx_.alloc(*S, R, maxld);
    S_ = std::move(S);
    pad_ = std::move(padv);
    key_++;  // a new layout: the captured graph is rebuilt
    np_ = np;
    SK_ = SK;
}

void SmolvlaTf::run(hipStream_t st) {
    Ctx c = ctx_;
    c.st = st;
    const int np = np_, C = C_, SK = SK_, H = H_, QF = nq_ * hd_, KV = nkv_ * hd_, W = QKVW_;
    const int EH = EH_, EF = EF_, F = F_;
    const float scale = 1.0f / std::sqrt((float)hd_);

    // row op feeding layer L: quantized in the same kernel for an int8 L, fp32
    // rows in f for an fp32 L
    auto rms_for = [&](const float* x, int rows, int H_, const float* w, float eps, const DLinear& L,
                       float* f) {
        RowQArgs r;
        r.op = 2;
        r.x = x;
        r.ldx = H_;
        r.w = w;
        r.eps = eps;
        r.rows = rows;
        r.H = H_;
        return rowop_for(c, L, r, L.int8() ? nullptr : f, H_, 0);
    };
    auto silu_for = [&](const float* gu_raw, int rows, int Fw, const DLinear& L) {
        RowQArgs r;
        r.op = 3;
        r.x = gu_raw;
        r.ldx = 2 * Fw;
        r.u = gu_raw + Fw;
        r.ldu = 2 * Fw;
        r.rows = rows;
        r.H = Fw;
        return rowop_for(c, L, r, L.int8() ? nullptr : gu_, Fw, 0);
    };

    // ---- prefix_forward (smollm2_lm.cpp:85-132)
    MaskSpec pm;
    pm.kind = 3;
    pm.n_groups = 4;
    pm.qg = pgroup_;
    pm.kg = pgroup_;
    pm.allow = pallow_;
    copy_f32(h_, prefix_in_, (int64_t)np * H, st);
    for (int L = 0; L < NL_; L++) {
        const VlmLayer& w = vlm_[L];
        float* buf = qkv_[L];
        const In xn = rms_for(h_, np, H, w.ln_in, eps_, w.qkv, xn_);
        if (L + 1 == NL_) {  // the last layer's K/V only (:107)
            linear(c, w.qkv, xn, buf + QF, W, np, 0, 0, QF, QF + 2 * KV);
            launch_rope_table(buf + QF, W, rope_p_, np, nkv_, hd_, st);
            break;
        }
        linear(c, w.qkv, xn, buf, W, np);
        launch_rope_table(buf, W, rope_p_, np, nq_ + nkv_, hd_, st);  // q and k heads
        attend(st, att_, QF, buf, W, buf + QF, W, buf + QF + KV, W, np, np, nq_, nkv_, hd_, scale, pm);
        linear(c, w.o, h_, H, att_, QF, np, 0, 1);
        const In x2 = rms_for(h_, np, H, w.ln_post, eps_, w.gu, xn_);
        linear(c, w.gu, x2, gu_raw_, 2 * F, np);
        const In g = silu_for(gu_raw_, np, F, w.down);
        linear(c, w.down, g, h_, H, np, 0, 1);
    }

    // ---- denoise (action_expert.cpp:325-395): cross-layer K/V re-projections once
    for (int L = 0; L < ENL_; L++) {
        const ExpLayer& w = exp_[L];
        if (w.self) continue;
        linear(c, w.k, ck_[L], KV, qkv_[L] + QF, W, np);
        linear(c, w.v, cv_[L], KV, qkv_[L] + QF + KV, W, np);
    }
    MaskSpec dm, cm;
    if (dcausal_) {
        dm.kind = 2;
        dm.causal_offset = np;
    } else {
        dm.kind = 1;
        dm.dense = dmask_;
        dm.ldm = SK;
        cm.kind = 1;
        cm.dense = cmask_;
        cm.ldm = np;
    }
    copy_f32(x_, noise_in_, (int64_t)C * mad_, st);
    const float dt = -1.0f / (float)steps_;
    for (int s = 0; s < steps_; s++) {
        // embed_suffix (:174-211)
        float* at = at_[s];
        linear(c, ain_, at, 2 * EH, x_, mad_, C);
        linear(c, at1_, mlp1_, EH, at, 2 * EH, C, 4);  // silu
        linear(c, at2_, eh_, EH, mlp1_, EH, C);
        for (int L = 0; L < ENL_; L++) {
            const ExpLayer& w = exp_[L];
            const In hn = rms_for(eh_, C, EH, w.ln_in, eeps_, w.q_or_qkv, ehn_);
            if (w.self) {
                float* buf = qkv_[L];
                float* suf = buf + (size_t)np * W;
                const RopeEpi rf{rope_full_, (enq_ + enkv_) * ehd_, ehd_};  // q and k heads
                linear(c, w.q_or_qkv, hn, suf, W, C, 0, 0, 0, -1, 1.0f, &rf);
                attend(st, att_, QF, suf, W, buf + QF, W, buf + QF + KV, W, C, SK, enq_, enkv_, ehd_,
                       scale, dm);
            } else {
                const RopeEpi rr{rope_reb_, enq_ * ehd_, ehd_};
                linear(c, w.q_or_qkv, hn, eq_, QF, C, 0, 0, 0, -1, 1.0f, &rr);
                attend(st, att_, QF, eq_, QF, ck_[L], KV, cv_[L], KV, C, np, enq_, enkv_, ehd_, scale, cm);
            }
            linear(c, w.o, eh_, EH, att_, QF, C, 0, 1);
            const In h2 = rms_for(eh_, C, EH, w.ln_post, eeps_, w.gu, ehn_);
            linear(c, w.gu, h2, gu_raw_, 2 * EF, C);
            const In g = silu_for(gu_raw_, C, EF, w.down);
            linear(c, w.down, g, eh_, EH, C, 0, 1);
        }
        launch_rmsnorm(hf_, eh_, out_norm_, C, EH, eeps_, st);
        if (rtc_) {  // v_t, its guidance, then the Euler step
            linear(c, aout_, v_, mad_, hf_, EH, C);
            const float time = (float)(1.0 + s * (-1.0 / steps_));
            launch_rtc_step(x_, v_, guide_, gweights_, gw_, s, C, mad_, time, dt, st);
        } else {
            linear(c, aout_, x_, mad_, hf_, EH, C, 0, 1, 0, -1, dt);  // x += dt * v_t
        }
    }
    copy_f32(act_out_, x_, (int64_t)C * mad_, st);
}

void SmolvlaTf::chunk_dev(const float* prefix, const int32_t* pad, int n_prefix, const float* noise,
                          float* actions, hipStream_t caller, const Rtc* rtc) {
    VLA_REQUIRE(prefix && pad && noise && actions, "smolvla: null buffer");
    VLA_REQUIRE(!rtc || (rtc->guide && rtc->weights && std::isfinite(rtc->max_guidance) && rtc->max_guidance > 0),
                "smolvla: guidance needs the guide, its weights and a positive finite max_guidance");
    ensure(pad, n_prefix);
    copy_f32(prefix_in_, prefix, (int64_t)n_prefix * H_, caller);
    copy_f32(noise_in_, noise, (int64_t)C_ * mad_, caller);
    rtc_ = rtc != nullptr;
    if (rtc_) {
        // the guidance weight per step, in the reference's float arithmetic
        // (its contracted s + tau * tau)
        gw_host_.assign(steps_, 0.0f);
        for (int s = 0; s < steps_; s++) {
            const double td = 1.0 + s * (-1.0 / steps_);
            const float tau = (float)(1.0 - td), sq = (1.0f - tau) * (1.0f - tau);
            gw_host_[s] = std::min((1.0f - tau) / tau * (std::fma(tau, tau, sq) / sq), rtc->max_guidance);
        }
        VLA_HIP_CHECK(hipMemcpyAsync(gw_, gw_host_.data(), steps_ * sizeof(float), hipMemcpyHostToDevice, caller));
        copy_f32(guide_, rtc->guide, (int64_t)C_ * mad_, caller);
        copy_f32(gweights_, rtc->weights, C_, caller);
    }
    (rtc_ ? replay_rtc_ : replay_).run(key_, own_, caller, [this](hipStream_t st) { run(st); });
    copy_f32(actions, act_out_, (int64_t)C_ * mad_, caller);
}

}  // namespace hip
}  // namespace vla
