// resnet.cpp - the ResNet-18 trunk on the device (see models.h).
//
// Follows src/models/act/resnet_backbone.cpp: load (<name>.meta / .bin, the
// block walk and its bounds, film_after), quantize_convs (the int8 stages),
// feat_size, and forward (stem, its GroupNorm, the max pool with the folded
// ReLU, then per block the downsample, conv1 + ReLU, conv2, and the residual
// add + ReLU or the FiLM point). The fp32 convolutions differ from the
// reference's packed-panel GEMM only by summation order; the int8 ones are
// conv2d_i8, bit-exact given the same input; the GroupNorm statistics are the
// reference's shifted sums in double (launch_groupnorm).
#include "ckpt.h"
#include "loader.h"
#include "models.h"

#include <algorithm>
#include <cstdlib>

namespace vla {
namespace hip {

namespace {
// VLA_HIP_CONV_FUSE=0 keeps the ReLU and the residual add + ReLU after each
// int8 conv as passes of their own (A/B runs; the values are the same bits)
bool conv_fuse_on() {
    const char* e = std::getenv("VLA_HIP_CONV_FUSE");
    return !(e && e[0] == '0' && e[1] == '\0');
}
// VLA_HIP_CONV_POOL_FUSE=0: the max pool as its own pass, the first block's
// first conv quantizing its output
bool conv_pool_fuse_on() {
    const char* e = std::getenv("VLA_HIP_CONV_POOL_FUSE");
    return !(e && e[0] == '0' && e[1] == '\0');
}
// VLA_HIP_CONV_SHARE=0: the block's first conv quantizes its input again
// after the downsample did
bool conv_share_on() {
    const char* e = std::getenv("VLA_HIP_CONV_SHARE");
    return !(e && e[0] == '0' && e[1] == '\0');
}
}  // namespace

ResNetTrunk::ResNetTrunk(const CkptFiles& files, const std::string& name, int in_h, int in_w, const TrunkOpts& o)
    : in_h_(in_h), in_w_(in_w) {
    const std::string bmeta = name + ".meta", bbin = name + ".bin";
    int in_ch = 3, stem_out = 64, stem_k = 7, stem_stride = 2, stem_pad = 3, gs = 0;
    struct BlockMeta {
        int cin, cout, stride, has_down;
    };
    std::vector<BlockMeta> bm;
    std::vector<int> film_after;
    // resnet_backbone.cpp:49-96
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
    for (const BlockMeta& b : bm)
        VLA_REQUIRE(shape_fits({b.cout, bk, bk, b.cin}) && shape_fits({b.cout, bk, bk, b.cout}) && b.stride >= 1 &&
                        (b.has_down == 0 || b.has_down == 1),
                    bmeta + ": invalid block (resnet_backbone.cpp:91-94 bounds)");
    gsize_ = gs;

    // <name>.bin: stem, then per block conv1, conv2, down (:96-154). Without
    // GroupNorm each conv is followed by its folded bias; with it, by the
    // norm's scale and bias (the conv has none).
    const std::vector<char> raw = files.bytes(bbin);
    VLA_REQUIRE(raw.size() % 4 == 0, bbin + ": size is not a whole number of floats");
    Floats take{reinterpret_cast<const float*>(raw.data()), raw.size() / 4};
    struct HostConv {
        const float *W, *b;
    };
    auto load_conv = [&](Conv& c, int cout, int k, int cin, int stride, int pad) {
        c.cout = cout;
        c.k = k;
        c.cin = cin;
        c.stride = stride;
        c.pad = pad;
        const size_t K = (size_t)k * k * cin;
        const float* W = take.take((size_t)cout * K, bbin.c_str());
        // rows padded to 4 floats (the stem's 147 -> 148), which the fp32
        // matrix-core GEMM needs; the pad is zero and the GEMM masks it anyway
        c.ldw = (int)((K + 3) & ~(size_t)3);
        if ((size_t)c.ldw == K) {
            c.W = A_.upload(W, (size_t)cout * K);
        } else {
            std::vector<float> padded((size_t)cout * c.ldw, 0.0f);
            for (int o = 0; o < cout; o++)
                std::copy(W + (size_t)o * K, W + (size_t)(o + 1) * K, padded.begin() + (size_t)o * c.ldw);
            c.W = A_.upload(padded.data(), padded.size());
        }
        if (!gs) {
            const float* b = take.take(cout, bbin.c_str());
            c.b = A_.upload(b, cout);
            return HostConv{W, b};
        }
        VLA_REQUIRE(cout % gs == 0 && cout / gs >= 1, bmeta + ": a conv's channels are not whole norm groups");
        VLA_REQUIRE(cout <= 1024 && gs <= 256, bmeta + ": GroupNorm wider than the device norm takes");
        c.gs = A_.upload(take.take(cout, bbin.c_str()), cout);
        c.gb = A_.upload(take.take(cout, bbin.c_str()), cout);
        return HostConv{W, nullptr};
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
    VLA_REQUIRE(take.done(), bbin + ": size does not match " + bmeta);
    int prev_idx = -1;
    for (int idx : film_after) {
        VLA_REQUIRE(idx >= 0 && idx < (int)blocks_.size() && idx > prev_idx,
                    bmeta + ": film_after must name blocks in ascending order");
        prev_idx = idx;
    }
    // FiLM points (film_total, resnet_backbone.cpp:190-195): block film_after[i]
    // reads gamma / beta at the sum of the earlier points' channels. A trunk
    // run without FiLM ignores the points the meta lists (ACT passes no
    // gamma / beta).
    film_off_.assign(blocks_.size(), -1);
    if (o.film)
        for (int idx : film_after) {
            film_off_[idx] = film_total_;
            film_total_ += blocks_[idx].c1.cout;
        }

    // feature grid (ResNetBackbone::feat_size, :197-209) and buffer sizes
    int h = conv_out(in_h_, stem_k, stem_stride, stem_pad), w = conv_out(in_w_, stem_k, stem_stride, stem_pad);
    const int h1 = h, w1 = w;
    h = conv_out(h, pool_k_, pool_stride_, pool_pad_);
    w = conv_out(w, pool_k_, pool_stride_, pool_pad_);
    const int ph = h, pw = w;
    VLA_REQUIRE(h1 > 0 && w1 > 0 && ph > 0 && pw > 0, bmeta + ": the image is smaller than the stem and pool");
    size_t map_max = std::max((size_t)h1 * w1 * stem_out, (size_t)ph * pw * stem_out), col_max = 0;
    // the im2col rows, then (64-float aligned) the split-K sums of the GEMM
    auto col_need = [&](const Conv& c, int H, int W) {
        const int Ho = conv_out(H, c.k, c.stride, c.pad), Wo = conv_out(W, c.k, c.stride, c.pad);
        const size_t npix = (size_t)Ho * Wo, K = (size_t)c.k * c.k * c.cin;
        const size_t rows = c.k == 1 && c.stride == 1 && c.pad == 0 ? 0 : col_rows_floats(npix, (int)K);
        col_max = std::max(col_max, rows + linear_f32_split_floats(Ho * Wo, c.cout, (int)K));
        if (gs) gw_doubles_ = std::max(gw_doubles_, groupnorm_work_doubles(Ho * Wo, c.cout));
    };
    col_need(stem_, in_h_, in_w_);
    int cmax = stem_out;
    for (const Block& blk : blocks_) {
        const int oh = conv_out(h, bk, blk.c1.stride, 1), ow = conv_out(w, bk, blk.c1.stride, 1);
        VLA_REQUIRE(oh > 0 && ow > 0, bmeta + ": the feature map vanishes inside the trunk");
        col_need(blk.c1, h, w);
        col_need(blk.c2, oh, ow);
        if (blk.has_down) col_need(blk.down, h, w);
        map_max = std::max(map_max, (size_t)oh * ow * blk.c1.cout);
        cmax = std::max(cmax, blk.c1.cout);
        h = oh;
        w = ow;
    }
    fh_ = h;
    fw_ = w;
    ch_ = blocks_.empty() ? stem_out : blocks_.back().c1.cout;

    // the int8 stages (quantize_convs, :169-188); Conv2d::init_int8 keeps a
    // conv fp32 unless Cout % 16 == 0 and K is within the int8 bound
    // (nn/conv.cpp:41-43)
    if (o.int8) {
        const int to = o.to < 0 ? (int)blocks_.size() + 1 : o.to;
        auto want = [&](int stage) { return stage >= o.from && stage < to; };
        auto quantize = [&](Conv& c, const HostConv& hc) {
            const int K = c.k * c.k * c.cin;
            if (c.cout % 16 || K > kMaxI8K) return;
            c.q8 = vla_linear_i8::from_f32(hc.W, hc.b, c.cout, K);
            n_int8_++;
        };
        if (want(0)) quantize(stem_, host[0]);
        size_t hi = 1;
        for (size_t i = 0; i < blocks_.size(); i++) {
            Block& blk = blocks_[i];
            const bool on = want((int)i + 1);
            if (on) quantize(blk.c1, host[hi]);
            if (on) quantize(blk.c2, host[hi + 1]);
            if (on && blk.has_down) quantize(blk.down, host[hi + 2]);
            hi += blk.has_down ? 3 : 2;
        }
    }

    a_ = A_.alloc<float>(map_max);
    b_ = A_.alloc<float>(map_max);
    c_ = A_.alloc<float>(map_max);
    res_ = A_.alloc<float>(map_max);
    col_ = A_.alloc<float>(col_max ? col_max : 4);
    col_floats_ = col_max;
    // up to 4096 maxima: a conv epilogue writes one per wave or block
    part_a_ = A_.alloc<float>(kConvPartsFused);
    part_b_ = A_.alloc<float>(kConvPartsFused);
    part_c_ = A_.alloc<float>(kConvPartsFused);
    if (film_total_) {
        film_g_ = A_.alloc<float>(film_total_);
        film_b_ = A_.alloc<float>(film_total_);
    }
    if (gs) {
        gA_ = A_.alloc<float>(cmax);
        gB_ = A_.alloc<float>(cmax);
        gW_ = A_.alloc<double>(gw_doubles_);
    }
    if (n_int8_) {
        size_t need = 0;
        auto ws = [&](const Conv& c, int H, int W) {
            if (c.q8) need = std::max(need, conv_shape(H, W, c.cin, c.k, c.stride, c.pad, c.cout).work);
        };
        h = in_h_;
        w = in_w_;
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
}

ConvArgs ResNetTrunk::i8_args(const Conv& c, const float* x, int H, int W, float* out, const float* in_part,
                              int in_nparts) const {
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
    return a;
}

int ResNetTrunk::conv(const Conv& c, const float* x, int H, int W, float* out, bool relu, hipStream_t st,
                      const float* in_part, int in_nparts, float* out_part, const float* resid, bool* resid_done,
                      int* xq_out, bool xq_in) {
    const int Ho = conv_out(H, c.k, c.stride, c.pad), Wo = conv_out(W, c.k, c.stride, c.pad);
    // GroupNorm after the conv: the conv itself runs without ReLU and the
    // norm applies it (resnet_backbone.cpp:218-262)
    const bool conv_relu = relu && !c.gs;
    int nparts = 0;
    if (c.q8) {
        ConvArgs a = i8_args(c, x, H, W, out, in_part, in_nparts);
        // the ReLU, or the residual add + ReLU, in the conv's epilogue
        const bool fuse_res = resid && !relu && !c.gs;
        if (out_part && (conv_relu || fuse_res) && conv_fuse_on()) {
            a.out_part = out_part;
            a.resid = fuse_res ? resid : nullptr;
        }
        a.xq_out = xq_out;
        a.xq_in = xq_in;
        const int fused = launch_conv2d_i8(a, st);
        if (fused > 0) {
            nparts = fused;
            if (fuse_res && resid_done) *resid_done = true;
        } else if (conv_relu) {
            // the relu pass writes the block maxima the next conv2d_i8 reads
            nparts = launch_relu_inplace(out, (int64_t)Ho * Wo * c.cout, st, out_part);
        }
    } else {
        const int K = c.k * c.k * c.cin;
        const float* rows = x;
        int ldx = K;
        const bool plain = c.k == 1 && c.stride == 1 && c.pad == 0;  // the map is already the GEMM's A
        // split-K sums after the im2col rows (the implicit form leaves those unused)
        const size_t rows_f = plain ? 0 : col_rows_floats((size_t)Ho * Wo, K);
        float* part = col_ + rows_f;
        const size_t part_f = col_floats_ - rows_f;
        if (plain || !launch_conv_f32_implicit(out, x, H, W, c.cin, c.k, c.stride, c.pad, Ho, Wo, c.W, c.b, c.cout,
                                               conv_relu ? 1 : 0, st, part, part_f)) {
            if (!plain) {
                ldx = (K + 3) & ~3;
                launch_im2col_f32(col_, ldx, x, H, W, c.cin, c.k, c.stride, c.pad, Ho, Wo, st);
                rows = col_;
            }
            launch_linear_f32(out, c.cout, rows, ldx, c.W, c.ldw, c.b, Ho * Wo, c.cout, K, conv_relu ? 1 : 0, 0, 1.0f, st,
                              part, part_f);
        }
    }
    if (c.gs)
        launch_groupnorm(out, out, c.gs, c.gb, Ho * Wo, c.cout, c.cout / gsize_, 1e-5f, relu, gA_, gB_, gW_,
                         gw_doubles_, st);
    return nparts;
}

// ResNetBackbone::forward (resnet_backbone.cpp:211-317); FiLM at the points
// film_off_ names (IMPACT)
//
// With int8 convolutions each conv2d_i8 input comes with the block maxima of
// |x| that its producer wrote where the producer can (the normalization, the
// max pool, the relu after conv1 when no GroupNorm follows it, the block's
// residual add + relu), so those convs run no absmax pass of their own; the
// maxima buffers follow the trunk buffers they describe. A GroupNorm output
// carries no maxima: the conv after it runs its absmax pass.
void ResNetTrunk::run(const float* x, const float* in_part, int in_nparts, float* out, hipStream_t st) {
    int h = conv_out(in_h_, stem_.k, stem_.stride, stem_.pad), w = conv_out(in_w_, stem_.k, stem_.stride, stem_.pad);
    const int ph = conv_out(h, pool_k_, pool_stride_, pool_pad_), pw = conv_out(w, pool_k_, pool_stride_, pool_pad_);
    float* B = b_;
    float* C = c_;
    float* pB = part_b_;
    float* pC = part_c_;
    int nB = 0;
    // With an int8 stem and an int8 first conv (no downsample, no GroupNorm)
    // the stem writes the maxima of max(0, out) and the max pool also leaves
    // its output's int8 map for that conv (xq_b), which then skips its own
    // quantization pass.
    bool xq_b = false;
    const Block* b0 = blocks_.empty() ? nullptr : &blocks_[0];
    if (stem_.q8 && !stem_.gs && b0 && !b0->has_down && b0->c1.q8 && !b0->c1.gs && conv_pool_fuse_on()) {
        ConvArgs sa = i8_args(stem_, x, in_h_, in_w_, a_, in_part, in_nparts);
        sa.out_part = pB;
        sa.relu_maxima = true;
        const int ns = launch_conv2d_i8(sa, st);
        if (ns > 0 && launch_conv_pool_quant(i8_args(b0->c1, B, ph, pw, a_, pB, ns), a_, h, w, pool_k_, pool_stride_,
                                             pool_pad_, st)) {
            nB = ns;
            xq_b = true;
        }
    } else {
        conv(stem_, x, in_h_, in_w_, a_, false, st, in_part, in_nparts);
    }
    if (!xq_b)
        nB = launch_maxpool_relu(B, a_, h, w, stem_.cout, pool_k_, pool_stride_, pool_pad_, ph, pw, st, pB,
                                 kConvPartsFused / 2);
    h = ph;
    w = pw;
    for (size_t bi = 0; bi < blocks_.size(); bi++) {
        const Block& blk = blocks_[bi];
        // the last block writes the trunk's output in place of a copy
        if (bi + 1 == blocks_.size()) C = out;
        const int oh = conv_out(h, blk.c1.k, blk.c1.stride, blk.c1.pad);
        const int ow = conv_out(w, blk.c1.k, blk.c1.stride, blk.c1.pad);
        const float* idn = B;
        // the downsample's int8 map of B serves the first conv too when both
        // are int8 over the same output grid (same input, maxima and scale)
        int xq = 0;
        if (blk.has_down) {
            conv(blk.down, B, h, w, res_, false, st, pB, nB, nullptr, nullptr, nullptr, &xq);
            idn = res_;
        }
        const bool share = xq && blk.c1.q8 && blk.down.q8 && nB > 0 && conv_share_on() &&
                           conv_out(h, blk.down.k, blk.down.stride, blk.down.pad) == oh &&
                           conv_out(w, blk.down.k, blk.down.stride, blk.down.pad) == ow;
        const int nA = conv(blk.c1, B, h, w, a_, true, st, pB, nB, part_a_, nullptr, nullptr, nullptr,
                            share || (bi == 0 && xq_b));
        const int fo = film_off_[bi];
        bool added = false;  // FiLM points keep their own pass
        const int nC = conv(blk.c2, a_, oh, ow, C, false, st, part_a_, nA, pC, fo < 0 ? idn : nullptr, &added);
        const int64_t n = (int64_t)oh * ow * blk.c1.cout;
        if (added) nB = nC;
        else
            nB = fo >= 0 ? launch_add_relu_film(C, idn, n, blk.c1.cout, film_g_ + fo, film_b_ + fo, st, pC)
                         : launch_add_relu(C, idn, n, st, pC);
        std::swap(B, C);
        std::swap(pB, pC);
        h = oh;
        w = ow;
    }
    if (B != out) copy_f32(out, B, (int64_t)fh_ * fw_ * ch_, st);
}

}  // namespace hip
}  // namespace vla
