// model_diffusion.cpp - Diffusion Policy end to end on the device (see models.h).
//
// Follows src/models/diffusion/diffusion_model.cpp (diffusion.meta, the
// DP_STEPS / DP_SCHEDULER / DIFFUSION_INT8 knobs, stats.bin, the frame cache,
// the conditioning layout, the executed slice and the MIN_MAX maps),
// unet1d.cpp (unet.bin's order, the blocks, the skips), rgb_encoder.cpp (the
// keypoint head and its grid) and scheduler.cpp (the beta schedules, the
// "leading" ladder and both reverse steps, in double on the host for the
// coefficients and on the device for the update). fp32 GEMMs differ from the
// reference's only by summation order; int8 ones are bit-exact given the same
// input rows.
#include "ckpt.h"
#include "loader.h"
#include "models.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <sstream>

namespace vla {
namespace hip {

namespace {

constexpr float kNormEps = 1e-8f;  // diffusion_model.cpp:18

// numpy.linspace as the reference builds the keypoint grid
// (rgb_encoder.cpp:14-28): start + i * step in double (fused, as the
// reference's -ffp-contract=fast build computes it), the endpoint pinned,
// then one cast to float
std::vector<float> np_linspace(double a, double b, int n) {
    std::vector<float> v((size_t)n);
    if (n == 1) {
        v[0] = (float)a;
        return v;
    }
    const double step = (b - a) / (double)(n - 1);
    for (int i = 0; i < n; i++) v[(size_t)i] = (float)std::fma(step, (double)i, a);
    v[(size_t)n - 1] = (float)b;
    return v;
}

// the Glide cosine alpha_bar of diffusers' squaredcos_cap_v2 schedule
double alpha_bar(double t) {
    const double c = std::cos((t + 0.008) / 1.008 * M_PI / 2.0);
    return c * c;
}

}  // namespace

DiffusionModel::Act DiffusionModel::act(int T, int C) {
    Act a;
    a.T = T;
    a.C = C;
    a.p = Ad_.alloc<float>((size_t)(T + 2 * P_) * C) + (size_t)P_ * C;  // zero rows stay zero
    return a;
}

DiffusionModel::DiffusionModel(const std::string& dir) {
    const CkptFiles files(dir);

    // diffusion.meta (diffusion_model.cpp:25-79)
    std::string sched = "DDPM", beta_schedule = "squaredcos_cap_v2", prediction = "epsilon";
    float beta_start = 1e-4f, beta_end = 0.02f;
    int resize_h = 0, resize_w = 0, film_scale = 1, clip = 1, separate = 1;
    std::vector<int> dd;
    const char* mf = "diffusion.meta";
    for (const auto& kv : files.meta_lines(mf)) {
        const std::string& k = kv.first;
        const std::string& v = kv.second;
        if (k == "n_obs_steps") read_values(mf, k, v, n_obs_);
        else if (k == "n_cams") read_values(mf, k, v, n_cams_);
        else if (k == "img_h") read_values(mf, k, v, img_h_);
        else if (k == "img_w") read_values(mf, k, v, img_w_);
        else if (k == "crop_h") read_values(mf, k, v, crop_h_);
        else if (k == "crop_w") read_values(mf, k, v, crop_w_);
        else if (k == "resize_h") read_values(mf, k, v, resize_h);
        else if (k == "resize_w") read_values(mf, k, v, resize_w);
        else if (k == "state_dim") read_values(mf, k, v, sd_);
        else if (k == "action_dim") read_values(mf, k, v, A_dim_);
        else if (k == "horizon") read_values(mf, k, v, H_);
        else if (k == "n_action_steps") read_values(mf, k, v, n_action_);
        else if (k == "num_keypoints") read_values(mf, k, v, kp_);
        else if (k == "kernel_size") read_values(mf, k, v, k_);
        else if (k == "n_groups") read_values(mf, k, v, groups_);
        else if (k == "step_embed_dim") read_values(mf, k, v, D_);
        else if (k == "num_train_timesteps") read_values(mf, k, v, n_train_);
        else if (k == "num_inference_steps") read_values(mf, k, v, n_infer_);
        else if (k == "beta_start") read_values(mf, k, v, beta_start);
        else if (k == "beta_end") read_values(mf, k, v, beta_end);
        else if (k == "beta_schedule") read_values(mf, k, v, beta_schedule);
        else if (k == "prediction_type") read_values(mf, k, v, prediction);
        else if (k == "clip_sample_range") read_values(mf, k, v, clip_range_);
        else if (k == "gn_eps") read_values(mf, k, v, gn_eps_);
        else if (k == "scheduler") read_values(mf, k, v, sched);
        else if (k == "film_scale") read_values(mf, k, v, film_scale);
        else if (k == "clip_sample") read_values(mf, k, v, clip);
        else if (k == "separate_encoders") read_values(mf, k, v, separate);
        else if (k == "down_dims") {
            std::istringstream ss(v);
            int w;
            while (ss >> w) dd.push_back(w);
            VLA_REQUIRE(ss.eof() && !dd.empty(), std::string(mf) + ": bad down_dims '" + v + "'");
        } else if (k == "cam") {
            std::string name;
            read_values(mf, k, v, name);
        }
    }
    down_dims_ = dd.empty() ? std::vector<int>{512, 1024, 2048} : dd;
    film_scale_ = film_scale != 0;
    clip_ = clip != 0;
    separate_ = separate != 0;
    VLA_REQUIRE(sched == "DDPM" || sched == "DDIM", "diffusion.meta: scheduler must be DDPM or DDIM");
    ddim_ = sched == "DDIM";
    // the step ablation's overrides (:81-90)
    const int steps_env = int_env("DP_STEPS", 0);
    if (steps_env > 0) n_infer_ = steps_env;
    if (const char* e = std::getenv("DP_SCHEDULER")) {
        const std::string s(e);
        VLA_REQUIRE(s == "DDIM" || s == "DDPM", "DP_SCHEDULER must be DDIM or DDPM");
        ddim_ = s == "DDIM";
    }

    // bounds (:92-106)
    VLA_REQUIRE(shape_fits({n_cams_, n_obs_, img_h_, img_w_, 3}) && shape_fits({sd_, n_obs_}) &&
                    shape_fits({H_, A_dim_}) && shape_fits({2, kp_, n_cams_, n_obs_}) &&
                    (long long)D_ + (long long)sd_ * n_obs_ + 2LL * kp_ * n_cams_ * n_obs_ <= INT_MAX &&
                    crop_h_ >= 0 && crop_w_ >= 0 && (crop_h_ == 0) == (crop_w_ == 0) && resize_h >= 0 &&
                    resize_w >= 0,
                "diffusion.meta: invalid shapes (diffusion_model.cpp:92-100 bounds)");
    VLA_REQUIRE(n_action_ > 0 && (long long)n_obs_ - 1 + n_action_ <= H_,
                "diffusion.meta: the executed slice runs past the horizon");
    VLA_REQUIRE(crop_h_ <= img_h_ && crop_w_ <= img_w_, "diffusion.meta: crop larger than the image");
    VLA_REQUIRE((resize_h == 0 || resize_h == img_h_) && (resize_w == 0 || resize_w == img_w_),
                "diffusion.meta: resizing is not supported (resize must equal the image size)");
    VLA_REQUIRE(n_infer_ <= n_train_, "diffusion.meta: more inference than training steps");

    // the noise schedule (DPNoiseScheduler::init, scheduler.cpp:21-67)
    VLA_REQUIRE(n_train_ > 0 && n_infer_ > 0, "diffusion: step counts must be positive");
    VLA_REQUIRE(!clip_ || (std::isfinite(clip_range_) && clip_range_ > 0), "diffusion: bad clip_sample_range");
    VLA_REQUIRE(prediction == "epsilon", "diffusion: only epsilon prediction is supported (scheduler.cpp:31)");
    std::vector<double> betas((size_t)n_train_);
    if (beta_schedule == "squaredcos_cap_v2") {
        for (int i = 0; i < n_train_; i++)
            betas[(size_t)i] =
                std::min(1.0 - alpha_bar((double)(i + 1) / n_train_) / alpha_bar((double)i / n_train_), 0.999);
    } else if (beta_schedule == "linear" || beta_schedule == "scaled_linear") {
        VLA_REQUIRE(beta_start > 0 && beta_start < 1 && beta_end > 0 && beta_end < 1,
                    "diffusion: beta_start / beta_end outside (0, 1)");
        const bool sq = beta_schedule == "scaled_linear";
        const double a = sq ? std::sqrt((double)beta_start) : (double)beta_start;
        const double b = sq ? std::sqrt((double)beta_end) : (double)beta_end;
        for (int i = 0; i < n_train_; i++) {
            const double v = a + (b - a) * (double)i / (double)std::max(n_train_ - 1, 1);
            betas[(size_t)i] = sq ? v * v : v;
        }
    } else {
        VLA_REQUIRE(false, "diffusion: unknown beta_schedule " + beta_schedule);
    }
    alphas_cumprod_.resize((size_t)n_train_);
    double run = 1.0;
    for (int i = 0; i < n_train_; i++) alphas_cumprod_[(size_t)i] = run *= 1.0 - betas[(size_t)i];
    const int ratio = n_train_ / n_infer_;  // "leading" spacing
    for (int i = n_infer_ - 1; i >= 0; i--) timesteps_.push_back(i * ratio);
    const int S = (int)timesteps_.size();

    // DIFFUSION_INT8 (:111-119)
    const int i8 = int_env("DIFFUSION_INT8", 0);

    // the rgb encoders (rgb_encoder.cpp:30-80), at the size they are fed
    oh_ = crop_h_ > 0 ? crop_h_ : img_h_;
    ow_ = crop_w_ > 0 ? crop_w_ : img_w_;
    const int dh = img_h_ - oh_, dw = img_w_ - ow_;  // the centre crop (:184-187)
    top_ = dh / 2 + ((dh & 3) == 3);
    left_ = dw / 2 + ((dw & 3) == 3);
    F_ = 2 * kp_;
    const int n_enc = separate_ ? n_cams_ : 1;
    size_t npx_max = 0, cmax = 0;
    for (int e = 0; e < n_enc; e++) {
        Encoder enc;
        const std::string nm = "rgb_encoder" + std::to_string(e);
        TrunkOpts to;
        to.int8 = (i8 & 2) != 0;
        enc.trunk = std::make_unique<ResNetTrunk>(files, nm + "_backbone", oh_, ow_, to);
        const int fh = enc.trunk->feat_h(), fw = enc.trunk->feat_w(), C = enc.trunk->channels();
        const std::vector<char> raw = files.bytes(nm + ".bin");
        VLA_REQUIRE(raw.size() % 4 == 0, nm + ".bin: size is not a whole number of floats");
        Floats take{reinterpret_cast<const float*>(raw.data()), raw.size() / 4};
        const float* kw = take.take((size_t)kp_ * C, (nm + ".bin").c_str());
        const float* kb = take.take(kp_, (nm + ".bin").c_str());
        const float* ow = take.take((size_t)F_ * F_, (nm + ".bin").c_str());
        const float* ob = take.take(F_, (nm + ".bin").c_str());
        VLA_REQUIRE(take.done(), nm + ".bin: size does not match num_keypoints and the trunk's channels");
        enc.kp.init(Ad_, kw, kb, kp_, C, false);
        enc.out.init(Ad_, ow, ob, F_, F_, false);
        const std::vector<float> px = np_linspace(-1.0, 1.0, fw), py = np_linspace(-1.0, 1.0, fh);
        std::vector<float> grid((size_t)fh * fw * 2);
        for (int y = 0; y < fh; y++)
            for (int x = 0; x < fw; x++) {
                grid[((size_t)y * fw + x) * 2] = px[(size_t)x];
                grid[((size_t)y * fw + x) * 2 + 1] = py[(size_t)y];
            }
        enc.grid = Ad_.upload(grid.data(), grid.size());
        npx_max = std::max(npx_max, (size_t)fh * fw);
        cmax = std::max(cmax, (size_t)fh * fw * C);
        enc_.push_back(std::move(enc));
    }

    // unet.bin (DPUNet1d::load, unet1d.cpp:36-145)
    const int nd = (int)down_dims_.size();
    G_ = (sd_ + n_cams_ * F_) * n_obs_;
    CD_ = D_ + G_;
    VLA_REQUIRE(nd <= 30 && groups_ > 0 && D_ >= 4 && D_ % 2 == 0 && shape_fits({4, D_, D_}) && k_ >= 1 &&
                    k_ % 2 == 1 && H_ > 0 && H_ % (1 << (nd - 1)) == 0 && std::isfinite(gn_eps_) && gn_eps_ > 0,
                "diffusion: invalid UNet shape (unet1d.cpp:38-43 bounds)");
    for (int w : down_dims_)
        VLA_REQUIRE(shape_fits({2, w, k_, w}) && w % groups_ == 0 && shape_fits({H_, w}) &&
                        shape_fits({2, w, CD_}),
                    "diffusion: invalid down_dims (unet1d.cpp:44-46 bounds)");
    for (int w : down_dims_)
        VLA_REQUIRE(w / groups_ <= kDpGnMaxGroup, "diffusion: norm groups wider than the device norm takes");
    // the final block normalizes in 8 groups whatever n_groups says (unet1d.cpp:301)
    VLA_REQUIRE(down_dims_[0] % 8 == 0 && down_dims_[0] / 8 <= kDpGnMaxGroup,
                "diffusion: down_dims[0] must split into the final block's 8 norm groups");
    const std::vector<char> raw = files.bytes("unet.bin");
    VLA_REQUIRE(raw.size() % 4 == 0, "unet.bin: size is not a whole number of floats");
    Floats take{reinterpret_cast<const float*>(raw.data()), raw.size() / 4};
    const bool q_unet = (i8 & 1) != 0;
    int ld_max = 64;
    // Linear::init + init_int8 (nn/linear.cpp:66): GEMM-role layers go int8
    // when N % 16 == 0 and K is within the int8 bound
    auto lin = [&](DLinear& L, int N, int K, bool gemm) {
        const float* W = take.take((size_t)N * K, "unet.bin");
        const float* b = take.take(N, "unet.bin");
        const bool q = q_unet && gemm && N % 16 == 0 && K <= kMaxI8K;
        L.init(Ad_, W, b, N, K, q);
        if (q) {
            n_int8_++;
            ld_max = std::max(ld_max, L.ldq());
        }
    };
    auto convb = [&](ConvB& cb, int cin, int cout, int kk) {
        cb.cin = cin;
        cb.cout = cout;
        lin(cb.L, cout, kk * cin, true);
        cb.gs = Ad_.upload(take.take(cout, "unet.bin"), cout);
        cb.gb = Ad_.upload(take.take(cout, "unet.bin"), cout);
    };
    std::vector<RowBlock> cond_rows;
    auto res = [&](Res& r, int cin, int cout) {
        r.cin = cin;
        r.cout = cout;
        convb(r.c1, cin, cout, k_);
        const int cn = film_scale_ ? 2 * cout : cout;
        const float* W = take.take((size_t)cn * CD_, "unet.bin");
        const float* b = take.take(cn, "unet.bin");
        cond_rows.push_back({W, b, cn});
        r.film_off = n_cond_;
        n_cond_ += cn;
        convb(r.c2, cout, cout, k_);
        r.has_res = cin != cout;
        if (r.has_res) lin(r.res, cout, cin, true);
    };
    DLinear step1, step2;
    lin(step1, 4 * D_, D_, false);
    lin(step2, D_, 4 * D_, false);
    std::vector<std::pair<int, int>> in_out{{A_dim_, down_dims_[0]}};
    for (int i = 0; i + 1 < nd; i++) in_out.emplace_back(down_dims_[(size_t)i], down_dims_[(size_t)i + 1]);
    down_.resize((size_t)nd);
    for (int i = 0; i < nd; i++) {
        Down& d = down_[(size_t)i];
        res(d.r1, in_out[(size_t)i].first, in_out[(size_t)i].second);
        res(d.r2, in_out[(size_t)i].second, in_out[(size_t)i].second);
        d.has = i + 1 < nd;
        if (d.has) lin(d.ds, in_out[(size_t)i].second, 3 * in_out[(size_t)i].second, true);
    }
    const int mid = down_dims_.back();
    res(mid1_, mid, mid);
    res(mid2_, mid, mid);
    up_.resize((size_t)nd - 1);
    for (int ind = 0; ind + 1 < nd; ind++) {
        // reversed(in_out[1:]): (dim_out, dim_in) pairs
        const int dim_out = in_out[(size_t)(nd - 1 - ind)].first, dim_in = in_out[(size_t)(nd - 1 - ind)].second;
        Up& u = up_[(size_t)ind];
        res(u.r1, dim_in * 2, dim_out);
        res(u.r2, dim_out, dim_out);
        u.has = ind < nd - 1;
        if (u.has) {
            // ConvTranspose1d(k 4, s 2, p 1), W [Cin = dim_out][4][Cout = dim_out]:
            // output row 2m = x[m-1] W[:,3,:] + x[m] W[:,1,:], row 2m+1 =
            // x[m] W[:,2,:] + x[m+1] W[:,0,:]; each is a GEMM over two
            // consecutive input rows, with the weights [Cout, 2 Cin]
            const int C = dim_out, uc = dim_out;
            u.uc = uc;
            const float* uw = take.take((size_t)C * 4 * uc, "unet.bin");
            const float* ub = take.take(uc, "unet.bin");
            std::vector<float> we((size_t)uc * 2 * C), wo((size_t)uc * 2 * C);
            for (int co = 0; co < uc; co++)
                for (int ci = 0; ci < C; ci++) {
                    auto w = [&](int kt) { return uw[((size_t)ci * 4 + kt) * uc + co]; };
                    we[(size_t)co * 2 * C + ci] = w(3);
                    we[(size_t)co * 2 * C + C + ci] = w(1);
                    wo[(size_t)co * 2 * C + ci] = w(2);
                    wo[(size_t)co * 2 * C + C + ci] = w(0);
                }
            u.even.init(Ad_, we.data(), ub, uc, 2 * C, false);
            u.odd.init(Ad_, wo.data(), ub, uc, 2 * C, false);
        }
    }
    convb(final_, down_dims_[0], down_dims_[0], k_);
    lin(final_conv_, A_dim_, down_dims_[0], false);
    VLA_REQUIRE(take.done(), "unet.bin: size does not match diffusion.meta");
    cond_.init(Ad_, cond_rows, CD_, false);

    // stats.bin (:121-164): state min / max, action min / max, per camera
    // image mean / std
    {
        const std::vector<char> st = files.bytes("stats.bin");
        const size_t n = (size_t)2 * sd_ + (size_t)2 * A_dim_ + (size_t)6 * n_cams_;
        VLA_REQUIRE(st.size() == n * 4, "stats.bin: size does not match the state, action and camera counts");
        const float* p = reinterpret_cast<const float*>(st.data());
        for (size_t i = 0; i < n; i++) VLA_REQUIRE(std::isfinite(p[i]), "stats.bin: non-finite value");
        for (int i = 0; i < sd_; i++) VLA_REQUIRE(p[sd_ + i] >= p[i], "stats.bin: state max below min");
        const float* a = p + 2 * sd_;
        bool degenerate = true;
        for (int i = 0; i < A_dim_; i++) {
            VLA_REQUIRE(a[A_dim_ + i] >= a[i], "stats.bin: action max below min");
            if (a[A_dim_ + i] - a[i] > 1e-6f) degenerate = false;
        }
        VLA_REQUIRE(!degenerate, "stats.bin: identity action statistics (every action range is empty)");
        std::vector<float> im((size_t)n_cams_ * 3), is((size_t)n_cams_ * 3);
        const float* c = p + 2 * sd_ + 2 * A_dim_;
        for (int cam = 0; cam < n_cams_; cam++)
            for (int i = 0; i < 3; i++) {
                im[(size_t)cam * 3 + i] = c[(size_t)cam * 6 + i];
                is[(size_t)cam * 3 + i] = c[(size_t)cam * 6 + 3 + i];
                VLA_REQUIRE(is[(size_t)cam * 3 + i] >= 0, "stats.bin: negative image std");
            }
        smin_ = Ad_.upload(p, sd_);
        smax_ = Ad_.upload(p + sd_, sd_);
        amin_ = Ad_.upload(a, A_dim_);
        amax_ = Ad_.upload(a + A_dim_, A_dim_);
        img_mean_ = Ad_.upload(im.data(), im.size());
        img_std_ = Ad_.upload(is.data(), is.size());
    }

    // activations: every layer output its own padded [T, C] rows, so the zero
    // rows around each stay zero and the taps views read them
    P_ = std::max(k_ / 2, 1);
    x0_ = act(H_, A_dim_);
    int T = H_;
    auto plan_res = [&](Res& r) {
        r.h = act(T, r.cout);
        r.o = act(T, r.cout);
    };
    const Act* x = &x0_;
    for (Down& d : down_) {
        plan_res(d.r1);
        plan_res(d.r2);
        x = &d.r2.o;
        if (d.has) {
            T /= 2;
            d.out = act(T, d.r2.cout);
            x = &d.out;
        }
    }
    plan_res(mid1_);
    plan_res(mid2_);
    x = &mid2_.o;
    for (int ind = 0; ind + 1 < nd; ind++) {
        Up& u = up_[(size_t)ind];
        const Act& skip = down_[(size_t)(nd - 1 - ind)].r2.o;
        VLA_REQUIRE(x->T == skip.T && x->C + skip.C == u.r1.cin, "diffusion: skip and upsampled shapes differ");
        u.cat = act(T, x->C + skip.C);
        plan_res(u.r1);
        plan_res(u.r2);
        x = &u.r2.o;
        if (u.has) {
            T *= 2;
            u.out = act(T, u.uc);
            x = &u.out;
        }
    }
    VLA_REQUIRE(T == H_, "diffusion: the UNet does not return to the horizon");
    // the 1x1 convs' outputs
    auto res_buf = [&](Res& r) {
        if (r.has_res) r.rb = Ad_.alloc<float>((size_t)r.o.T * r.cout);
    };
    for (Down& d : down_) {
        res_buf(d.r1);
        res_buf(d.r2);
    }
    res_buf(mid1_);
    res_buf(mid2_);
    for (Up& u : up_) {
        res_buf(u.r1);
        res_buf(u.r2);
    }
    // the concatenations [x | skip] are written by their producers: the skip
    // by its level's last block norm, x by the mid block's last norm or the
    // previous transposed conv
    for (int ind = 0; ind + 1 < nd; ind++) {
        Up& u = up_[(size_t)ind];
        Res& skip = down_[(size_t)(nd - 1 - ind)].r2;
        skip.out2 = u.cat.p + (u.cat.C - skip.cout);
        skip.ldo2 = u.cat.C;
        if (ind == 0) {
            mid2_.out2 = u.cat.p;
            mid2_.ldo2 = u.cat.C;
        }
        if (u.has) {
            const bool next = ind + 2 < nd;
            u.up_to = next ? up_[(size_t)ind + 1].cat.p : u.out.p;
            u.up_ld = next ? up_[(size_t)ind + 1].cat.C : u.uc;
        }
    }
    f_ = act(H_, down_dims_[0]);
    eps_ = Ad_.alloc<float>((size_t)H_ * A_dim_);

    // the time embedding of every step, through step1 -> mish -> step2, then
    // the cond encoders' mish (DPUNet1d::step_embedding and forward,
    // unet1d.cpp:213-240)
    ctx_.alloc(Ad_, std::max(H_, 1), ld_max);
    hipStream_t st = library_stream();
    {
        const int half = D_ / 2;
        const float sc = std::log(10000.0f) / (float)(half - 1);
        std::vector<float> emb((size_t)S * D_);
        for (int i = 0; i < S; i++)
            for (int j = 0; j < half; j++) {
                const float f = (float)timesteps_[(size_t)i] * std::exp(-(float)j * sc);
                emb[(size_t)i * D_ + j] = std::sin(f);
                emb[(size_t)i * D_ + half + j] = std::cos(f);
            }
        DeviceArena tmp;
        float* e = tmp.upload(emb.data(), emb.size());
        float* wide = tmp.alloc<float>((size_t)S * 4 * D_);
        temb_ = Ad_.alloc<float>((size_t)S * D_);
        Ctx c = ctx_;
        c.st = st;
        linear(c, step1, wide, 4 * D_, e, D_, S);
        launch_mish(wide, (int64_t)S * 4 * D_, st);
        linear(c, step2, temb_, D_, wide, 4 * D_, S);
        launch_mish(temb_, (int64_t)S * D_, st);
        VLA_HIP_CHECK(hipStreamSynchronize(st));
    }

    // per-query buffers
    const size_t px = (size_t)img_h_ * img_w_ * 3;
    const int slots = n_obs_ * n_cams_;
    frames_ = Ad_.alloc<uint8_t>((size_t)slots * px);
    norm_ = Ad_.alloc<float>((size_t)oh_ * ow_ * 3);
    fmap_ = Ad_.alloc<float>(cmax);
    kpmap_ = Ad_.alloc<float>(npx_max * kp_);
    kpts_ = Ad_.alloc<float>(F_);
    feats_ = Ad_.alloc<float>((size_t)slots * F_);
    state_ = Ad_.alloc<float>((size_t)n_obs_ * sd_);
    noise_ = Ad_.alloc<float>((size_t)(1 + S) * H_ * A_dim_);
    gcond_ = Ad_.alloc<float>(G_);
    gm_ = Ad_.alloc<float>((size_t)S * CD_);
    cond_all_ = Ad_.alloc<float>((size_t)S * n_cond_);
    act_out_ = Ad_.alloc<float>((size_t)n_action_ * A_dim_);
    slot_px_.resize((size_t)slots);
    for (int i = 0; i < slots; i++) enc_replay_.push_back(std::make_unique<GraphReplay>());
    VLA_HIP_CHECK(hipStreamCreateWithFlags(&own_, hipStreamNonBlocking));
}

DiffusionModel::~DiffusionModel() {
    if (own_) (void)hipStreamDestroy(own_);
}

int DiffusionModel::int8_convs() const {
    int n = 0;
    for (const Encoder& e : enc_) n += e.trunk->int8_convs();
    return n;
}

// out rows [rows, L.N] = the k-tap convolution of x (zero padding pad = k/2
// for stride 1, 1 for the strided downsample): row t reads the k * C floats
// from x row t * stride - pad on
void DiffusionModel::conv(const Ctx& c, const DLinear& L, const Act& x, int k, int stride, float* out, int ldo,
                          int rows) const {
    const int pad = stride == 1 ? k / 2 : 1;
    VLA_REQUIRE(L.K == k * x.C && pad <= P_ && (rows - 1) * stride - pad + k <= x.T + P_,
                "diffusion: a convolution reads past its sequence's zero rows");
    In in;
    in.f = x.p - (size_t)pad * x.C;
    in.ldf = stride * x.C;
    in.taps = in.ldf < L.K;
    linear(c, L, in, out, ldo, rows);
}

// DPResBlock::forward (unet1d.cpp:176-211): conv1 -> GN -> Mish -> FiLM,
// conv2 -> GN -> Mish, + the residual: x, or the 1x1 conv of x when the
// width changes, run before the second norm, which adds its output (the
// reference's out[i] += r[i], the same sum)
void DiffusionModel::res_block(const Ctx& c, const Res& r, const Act& x, int step) const {
    const int T = x.T, C = r.cout;
    conv(c, r.c1.L, x, k_, 1, r.h.p, C, T);
    const float* film = cond_all_ + (size_t)step * n_cond_ + r.film_off;
    launch_dp_gn_mish(r.h.p, C, r.h.p, C, T, C, groups_, r.c1.gs, r.c1.gb, gn_eps_, film_scale_ ? film : nullptr,
                      film_scale_ ? film + C : film, nullptr, 0, c.st);
    conv(c, r.c2.L, r.h, k_, 1, r.o.p, C, T);
    if (r.has_res) linear(c, r.res, r.rb, C, x.p, x.C, T);  // x W^T + b
    launch_dp_gn_mish(r.o.p, C, r.o.p, C, T, C, groups_, r.c2.gs, r.c2.gb, gn_eps_, nullptr, nullptr,
                      r.has_res ? r.rb : x.p, r.has_res ? C : x.C, c.st, r.out2, r.ldo2);
}

// DPUNet1d::forward (unet1d.cpp:227-303) for sampler step `step`: x0_ -> eps_
void DiffusionModel::unet(const Ctx& c, int step) const {
    const int nd = (int)down_.size();
    const Act* x = &x0_;
    for (const Down& d : down_) {
        res_block(c, d.r1, *x, step);
        res_block(c, d.r2, d.r1.o, step);
        x = &d.r2.o;
        if (d.has) {
            conv(c, d.ds, d.r2.o, 3, 2, d.out.p, d.out.C, d.out.T);
            x = &d.out;
        }
    }
    res_block(c, mid1_, *x, step);
    res_block(c, mid2_, mid1_.o, step);
    x = &mid2_.o;
    for (int ind = 0; ind + 1 < nd; ind++) {
        const Up& u = up_[(size_t)ind];
        // u.cat already holds [x | skip]: their producers wrote it
        res_block(c, u.r1, u.cat, step);
        res_block(c, u.r2, u.r1.o, step);
        x = &u.r2.o;
        if (u.has) {
            const Act& b = u.r2.o;
            In ev;
            ev.f = b.p - b.C;
            ev.ldf = b.C;
            ev.taps = true;
            linear(c, u.even, ev, u.up_to, 2 * u.up_ld, b.T);
            In od = ev;
            od.f = b.p;
            linear(c, u.odd, od, u.up_to + u.up_ld, 2 * u.up_ld, b.T);
            x = &u.out;
        }
    }
    const int C0 = down_dims_[0];
    conv(c, final_.L, *x, k_, 1, f_.p, C0, H_);
    launch_dp_gn_mish(f_.p, C0, f_.p, C0, H_, C0, 8, final_.gs, final_.gb, gn_eps_, nullptr, nullptr, nullptr, 0,
                      c.st);
    linear(c, final_conv_, eps_, A_dim_, f_.p, C0, H_);
}

// the conditioning, the FiLM vectors of every step, the prior, then every
// UNet pass and reverse step (DiffusionModel::predict, :249-262, and
// DPNoiseScheduler::step)
void DiffusionModel::sample(hipStream_t st) {
    Ctx c = ctx_;
    c.st = st;
    const int S = (int)timesteps_.size(), n = H_ * A_dim_;
    launch_dp_gcond(gcond_, state_, smin_, smax_, feats_, n_obs_, sd_, n_cams_, F_, kNormEps, st);
    launch_dp_cond_rows(gm_, temb_, gcond_, S, D_, G_, st);
    linear(c, cond_, cond_all_, n_cond_, gm_, CD_, S);
    copy_f32(x0_.p, noise_, n, st);
    for (int i = 0; i < S; i++) {
        unet(c, i);
        const int t = timesteps_[(size_t)i];
        const int prev = ddim_ ? t - n_train_ / n_infer_ : (i + 1 < S ? timesteps_[(size_t)i + 1] : -1);
        const double ap = alphas_cumprod_[(size_t)t];
        const double app = prev >= 0 ? alphas_cumprod_[(size_t)prev] : 1.0;
        const double bp = 1.0 - ap;
        double c0, c1, var = 0.0;
        if (ddim_) {
            c0 = std::sqrt(app);
            c1 = std::sqrt(std::max(0.0, 1.0 - app));
        } else {
            const double cur_a = ap / app, cur_b = 1.0 - cur_a;
            c0 = (std::sqrt(app) * cur_b) / bp;
            c1 = std::sqrt(cur_a) * (1.0 - app) / bp;
            if (t > 0) var = std::sqrt(std::max((1.0 - app) / (1.0 - ap) * cur_b, 1e-20));
        }
        const float* z = !ddim_ && t > 0 ? noise_ + (size_t)(i + 1) * n : nullptr;
        launch_dp_sched_step(x0_.p, eps_, z, n, std::sqrt(ap), std::sqrt(bp), c0, c1, var, ddim_, clip_,
                             (double)clip_range_, st);
    }
}

// DPRgbEncoder::forward (rgb_encoder.cpp:82-96) of slot (step, camera)'s frame
void DiffusionModel::encode(int slot, hipStream_t st) {
    const int cam = slot % n_cams_;
    Encoder& e = enc_[(size_t)(separate_ ? cam : 0)];
    const size_t px = (size_t)img_h_ * img_w_ * 3;
    launch_crop_normalize(norm_, frames_ + (size_t)slot * px, img_h_, img_w_, top_, left_, oh_, ow_,
                          img_mean_ + cam * 3, img_std_ + cam * 3, kNormEps, st);
    e.trunk->run(norm_, nullptr, 0, fmap_, st);
    Ctx c = ctx_;
    c.st = st;
    const int npx = e.trunk->feat_h() * e.trunk->feat_w();
    linear(c, e.kp, kpmap_, kp_, fmap_, e.trunk->channels(), npx);
    launch_spatial_softmax(kpts_, kpmap_, e.grid, npx, kp_, st);
    linear(c, e.out, feats_ + (size_t)slot * F_, F_, kpts_, F_, 1, 1);  // Linear + ReLU
}

void DiffusionModel::predict(const uint8_t* frames, const float* state, const float* noise, bool unnormalize,
                             float* actions) {
    VLA_REQUIRE(frames && state && actions, "diffusion: null buffer");
    hipStream_t st = library_stream();
    const int S = (int)timesteps_.size(), n = H_ * A_dim_;
    VLA_HIP_CHECK(hipMemcpyAsync(state_, state, (size_t)n_obs_ * sd_ * 4, hipMemcpyHostToDevice, st));
    if (noise)
        VLA_HIP_CHECK(hipMemcpyAsync(noise_, noise, (size_t)(1 + S) * n * 4, hipMemcpyHostToDevice, st));
    else
        VLA_HIP_CHECK(hipMemsetAsync(noise_, 0, (size_t)(1 + S) * n * 4, st));
    // the frame cache (diffusion_model.cpp:224-246): a frame equal to one a
    // slot of the same camera holds reuses that slot's features
    const size_t px = (size_t)img_h_ * img_w_ * 3;
    for (int s = 0; s < n_obs_; s++)
        for (int cam = 0; cam < n_cams_; cam++) {
            const int slot = s * n_cams_ + cam;
            const uint8_t* f = frames + (size_t)slot * px;
            int hit = -1;
            for (int k = 0; k < n_obs_ && hit < 0; k++) {
                const std::vector<uint8_t>& p = slot_px_[(size_t)(k * n_cams_ + cam)];
                if (p.size() == px && !std::memcmp(p.data(), f, px)) hit = k * n_cams_ + cam;
            }
            if (hit >= 0) {
                if (hit != slot) copy_f32(feats_ + (size_t)slot * F_, feats_ + (size_t)hit * F_, F_, st);
            } else {
                VLA_HIP_CHECK(hipMemcpyAsync(frames_ + (size_t)slot * px, f, px, hipMemcpyHostToDevice, st));
                enc_replay_[(size_t)slot]->run(1, own_, st, [this, slot](hipStream_t s2) { encode(slot, s2); });
            }
            if (hit != slot) slot_px_[(size_t)slot].assign(f, f + px);
        }
    replay_.run(1, own_, st, [this](hipStream_t s2) { sample(s2); });
    launch_dp_actions(act_out_, x0_.p, n_obs_ - 1, n_action_, A_dim_, amin_, amax_, kNormEps, unnormalize, st);
    VLA_HIP_CHECK(hipMemcpyAsync(actions, act_out_, (size_t)n_action_ * A_dim_ * 4, hipMemcpyDeviceToHost, st));
    VLA_HIP_CHECK(hipStreamSynchronize(st));
}

}  // namespace hip
}  // namespace vla
