// models.h - the policy graphs of the reference on the device: the ACT
// transformer, the Octo block transformer, the SmolVLA action chunk (SmolLM2
// prefix + action expert flow-matching denoise) and SmolVLA's SigLIP vision
// tower. Each loads the reference's own
// .meta/.bin checkpoint layout, holds its weights in HBM (int8 rows + scales for
// the layers its int8 mask selects, fp32 otherwise), and runs a whole forward
// pass as one HIP graph on inputs already on the device.
#pragma once

#include "graph.h"
#include "tokenizer.h"

#include <map>
#include <memory>
#include <string>
#include <vector>

namespace vla {
namespace hip {

class CkptFiles;

// ------------------------------------------------------------------- ACT --
// src/models/act/act_transformer.{h,cpp}: DETR-style post-norm encoder over
// [latent | state | camera tokens], decoder with `chunk` zero-initialised
// queries, final LayerNorm and an fp32 action head. int8 mask bits as
// act_transformer.cpp:27 (1 encoder attention, 2 w1, 4 w2, 8 img_proj,
// 16 decoder).
//
// IMPACT (src/models/impact/impact_model.cpp:59-68) drives the same
// transformer with int8_state (the state projection joins the img_proj int8
// group, act_transformer.cpp:127-130) and a text tail: up to act.meta's n_text
// tokens of its T5 tower appended after the camera tokens, their positions
// after the camera positions (build_tokens, :212-250).
class ActTf {
public:
    // tag names the files: <tag>.meta / <tag>.bin ("act", IMPACT's "impact")
    ActTf(const std::string& dir, int img_ch, int int8_mask, bool int8_state = false,
          const std::string& tag = "act");
    ~ActTf();
    int chunk() const { return chunk_; }
    int action_dim() const { return action_dim_; }
    int state_dim() const { return state_dim_; }
    int dim() const { return d_; }
    int img_ch() const { return img_ch_; }
    int n_tokens(int n_cams, int fh, int fw, int nt = 0) const { return n_1d_ + n_cams * fh * fw + nt; }
    int n_text() const { return n_text_; }
    int int8_layers() const { return n_int8_; }
    // device pointers; feats [n_cams * fh * fw, img_ch], state_norm [state_dim],
    // actions_norm [chunk, action_dim]
    void forward_dev(const float* feats, int n_cams, int fh, int fw, const float* state_norm,
                     float* actions_norm, hipStream_t caller) {
        forward_text_dev(feats, n_cams, fh, fw, state_norm, nullptr, nullptr, 0, actions_norm, caller);
    }
    // with the text tail: text / text_pos [n_text_real, dim] (device), of which
    // min(max(n_text_real, 0), n_text) rows enter the sequence (clamp_text)
    void forward_text_dev(const float* feats, int n_cams, int fh, int fw, const float* state_norm,
                          const float* text, const float* text_pos, int n_text_real, float* actions_norm,
                          hipStream_t caller);
    int graph_nodes() const { return replay_.nodes(); }

private:
    struct Enc {
        DLinear qk, v, o, w1, w2;
        const float *n1s, *n1b, *n2s, *n2b;
    };
    struct Dec {
        DLinear sqk, sv, so, cq, ck, cv, co, w1, w2;
        const float *n1s, *n1b, *n2s, *n2b, *n3s, *n3b;
    };
    void ensure(int n_cams, int fh, int fw, int nt);
    // the whole forward, or (head_only) decoder layer 0's self-attention block
    // and norm1 alone, which read only the zero queries, dec_pos and weights
    void run(hipStream_t st, bool head_only = false);

    int d_ = 512, heads_ = 8, hd_ = 64, ff_ = 3200, n_enc_ = 4, n_dec_ = 1, chunk_ = 100;
    int state_dim_ = 6, action_dim_ = 6, n_1d_ = 2, img_ch_ = 0, n_int8_ = 0, n_text_ = 0;
    float eps_ = 1e-5f;
    DeviceArena A_;
    DLinear img_proj_, state_proj_, head_;
    const float *latent_ = nullptr, *pos1d_ = nullptr, *dec_pos_ = nullptr, *dec_ns_ = nullptr,
                *dec_nb_ = nullptr;
    std::vector<Enc> enc_;
    std::vector<Dec> dec_;
    // per-shape state
    int n_cams_ = -1, fh_ = -1, fw_ = -1, nt_ = -1, T_ = 0;
    std::unique_ptr<DeviceArena> S_;
    float *feats_ = nullptr, *state_ = nullptr, *act_out_ = nullptr, *x_ = nullptr, *pos_ = nullptr,
          *xp_ = nullptr, *qk_ = nullptr, *v_ = nullptr, *att_ = nullptr, *ff_buf_ = nullptr,
          *dx_ = nullptr, *zero_ = nullptr, *kpos_ = nullptr, *ckb_ = nullptr, *cvb_ = nullptr,
          *dq_ = nullptr, *text_ = nullptr;
    Ctx ctx_;
    hipStream_t own_ = nullptr;
    GraphReplay replay_;
    // decoder layer 0 after its self-attention block and norm1, computed once
    // by run(st, true) (same kernels, same bits) and copied in per forward:
    // dx, and the cross-query input (fp32 rows, or their int8 slot bytes)
    float *head_dx_ = nullptr, *head_xp_ = nullptr, *head_qs_ = nullptr;
    int8_t* head_q_ = nullptr;
    size_t head_q_bytes_ = 0;
    bool head_done_ = false;
};

// ------------------------------------------------------- ResNet-18 trunk --
// src/models/act/resnet_backbone.{h,cpp}: <name>.meta / .bin, a 7x7/s2 stem,
// a max pool with the folded ReLU, basic blocks, on one normalized NHWC image
// at a time. BatchNorm folded into conv biases (ACT, IMPACT), or GroupNorm
// after every conv (gn_group_size channels per group: Diffusion Policy's
// encoders; the convs then carry no bias). fp32 convs are the implicit GEMM
// or im2col + the fp32 matrix-core linear; int8 ones are conv2d_i8, bit-exact
// to the reference's Conv2d int8 path given the same input. FiLM points
// (film_after) modulate block outputs when the options ask for them.
struct TrunkOpts {
    bool film = false;       // apply (1 + gamma) relu(v) + beta at film_after
    bool int8 = false;       // convs of stages [from, to) through conv2d_i8
    int from = 0, to = -1;   // stage 0 the stem, 1.. the blocks; to < 0: all
};

class ResNetTrunk {
public:
    ResNetTrunk(const CkptFiles& files, const std::string& name, int in_h, int in_w, const TrunkOpts& o);
    int feat_h() const { return fh_; }
    int feat_w() const { return fw_; }
    int channels() const { return ch_; }
    int int8_convs() const { return n_int8_; }
    bool stem_int8() const { return stem_.q8 != nullptr; }
    int film_total() const { return film_total_; }
    float* film_gamma() const { return film_g_; }
    float* film_beta() const { return film_b_; }
    // x [in_h, in_w, 3] normalized; in_part / in_nparts: block maxima of |x|
    // (for an int8 stem; nparts 0 runs its absmax pass); out [fh * fw, C]
    void run(const float* x, const float* in_part, int in_nparts, float* out, hipStream_t st);

private:
    struct Conv {
        int cin = 0, cout = 0, k = 0, stride = 1, pad = 0;
        int ldw = 0;         // W's row stride: k * k * cin rounded up to 4 (zero pad)
        float* W = nullptr;  // fp32 [cout, ldw]
        float* b = nullptr;  // [cout], null under GroupNorm
        const float *gs = nullptr, *gb = nullptr;  // GroupNorm scale / bias [cout]
        std::unique_ptr<vla_linear_i8> q8;  // conv2d_i8 weights when the stage is int8
    };
    struct Block {
        Conv c1, c2, down;
        bool has_down = false;
    };
    // out [Hout * Wout, cout] = conv(x [H, W, cin]), then its GroupNorm (if
    // any) and the ReLU (relu). int8 convs: in_part / in_nparts are the block
    // maxima of |x| its producer wrote, out_part receives those of the relu'd
    // output; returns their count (0 when none are written). The ReLU runs
    // in the conv's epilogue where its kernel fuses it, else as a pass. resid
    // (an int8 conv without ReLU or GroupNorm): the block's residual, added
    // and ReLU'd in the epilogue where the kernel fuses that (*resid_done =
    // true, the maxima then those of the sum); otherwise the caller adds it.
    // ConvArgs of an int8 conv over x [H, W, cin] into out, with the trunk's workspace
    ConvArgs i8_args(const Conv& c, const float* x, int H, int W, float* out, const float* in_part,
                     int in_nparts) const;
    // xq_out / xq_in: ConvArgs' shared int8 map of x (the downsample, then
    // the block's first conv over the same input and output grid).
    int conv(const Conv& c, const float* x, int H, int W, float* out, bool relu, hipStream_t st,
             const float* in_part = nullptr, int in_nparts = 0, float* out_part = nullptr,
             const float* resid = nullptr, bool* resid_done = nullptr, int* xq_out = nullptr, bool xq_in = false);

    int in_h_ = 0, in_w_ = 0, gsize_ = 0;
    int pool_k_ = 3, pool_stride_ = 2, pool_pad_ = 1;
    std::vector<int> film_off_;  // per block, its point's offset in gamma / beta, or -1
    int film_total_ = 0;
    float *film_g_ = nullptr, *film_b_ = nullptr;
    int fh_ = 0, fw_ = 0, ch_ = 0, n_int8_ = 0;
    DeviceArena A_;
    Conv stem_;
    std::vector<Block> blocks_;
    // the activation maps (reused image after image), the im2col rows +
    // split-K sums, the conv2d_i8 workspace, the GroupNorm affine and sums
    float *a_ = nullptr, *b_ = nullptr, *c_ = nullptr, *res_ = nullptr, *col_ = nullptr;
    float *part_a_ = nullptr, *part_b_ = nullptr, *part_c_ = nullptr;
    size_t col_floats_ = 0;
    void* work_ = nullptr;
    size_t work_bytes_ = 0;
    float *gA_ = nullptr, *gB_ = nullptr;
    double* gW_ = nullptr;
    size_t gw_doubles_ = 0;
};

// What tells an ACT-shaped model's files and knobs apart: ACT itself, or
// IMPACT (impact_model.cpp:50-66: the trunk in vision.meta/.bin, the
// transformer in impact.meta/.bin with int8_state, IMPACT_INT8 and its conv
// range, FiLM points in the trunk).
struct ActSpec {
    const char* backbone = "backbone";
    const char* tf = "act";
    const char* int8_env = "ACT_INT8";
    const char* conv_from_env = "ACT_I8_CONV_FROM";
    const char* conv_to_env = "ACT_I8_CONV_TO";
    bool int8_state = false;
    bool film = false;  // the trunk applies (1 + gamma) relu(v) + beta at film_after
};

// ------------------------------------------------------------ ACT policy --
// src/models/act/act_model.{h,cpp} + resnet_backbone.{h,cpp}: uint8 camera
// frames -> per-camera normalization -> ResNet-18 trunk (BatchNorm folded into
// conv biases, 7x7/s2 stem, 3x3/s2 max pool with the folded ReLU, basic
// blocks) -> ActTf -> action un-normalization. Files: config.txt,
// backbone.meta/.bin, act.meta/.bin, stats.bin (a directory or a vla.simd
// GGUF carrying them). ACT_INT8 is read at load as act_model.cpp:57-64 reads
// it: bits 1..16 pick the transformer's int8 layers, bit 32 routes the
// backbone convs of stages [ACT_I8_CONV_FROM, ACT_I8_CONV_TO) through
// conv2d_i8 (stage 0 the stem, 1.. the blocks). With an IMPACT spec the
// FiLM points of the trunk modulate the block outputs (resnet_backbone.cpp:
// 259-290) and the transformer takes IMPACT's text tail.
class ActModel {
public:
    explicit ActModel(const std::string& dir, const ActSpec& spec = ActSpec{});
    ~ActModel();
    int chunk() const { return tf_->chunk(); }
    int action_dim() const { return tf_->action_dim(); }
    int state_dim() const { return tf_->state_dim(); }
    int n_cams() const { return n_cams_; }
    int img_h() const { return img_h_; }
    int img_w() const { return img_w_; }
    int feat_h() const { return trunk_->feat_h(); }
    int feat_w() const { return trunk_->feat_w(); }
    int feat_ch() const { return trunk_->channels(); }
    int int8_convs() const { return trunk_->int8_convs(); }
    int int8_layers() const { return tf_->int8_layers(); }
    int graph_nodes() const { return replay_.nodes() + tf_->graph_nodes(); }
    // device pointers: images [n_cams, img_h, img_w, 3] uint8, state
    // [state_dim] raw, actions [chunk, action_dim]
    void predict_dev(const uint8_t* images, const float* state, bool unnormalize, float* actions,
                     hipStream_t caller) {
        predict_text_dev(images, state, nullptr, nullptr, 0, unnormalize, actions, caller);
    }
    // with IMPACT's text tail (device text / text_pos [n_text, dim], of which
    // n_text_real rows enter the sequence; act_transformer.cpp:343-360)
    void predict_text_dev(const uint8_t* images, const float* state, const float* text, const float* text_pos,
                          int n_text_real, bool unnormalize, float* actions, hipStream_t caller);
    // FiLM (spec.film): the trunk's gamma / beta device buffers [film_total],
    // the points concatenated in film_after order, which the caller fills
    int film_total() const { return trunk_->film_total(); }
    float* film_gamma() const { return trunk_->film_gamma(); }
    float* film_beta() const { return trunk_->film_beta(); }
    int tf_dim() const { return tf_->dim(); }
    int tf_n_text() const { return tf_->n_text(); }
    // the backbone alone (encode_view per camera): feats [n_cams * fh * fw, C]
    void encode_dev(const uint8_t* images, float* feats, hipStream_t caller);

private:
    void run_backbone(hipStream_t st, const uint8_t* images, float* feats);

    int img_h_ = 480, img_w_ = 640, n_cams_ = 2;
    float norm_eps_ = 1e-8f;
    DeviceArena A_;
    std::unique_ptr<ResNetTrunk> trunk_;
    std::unique_ptr<ActTf> tf_;
    float *img_mean_ = nullptr, *img_std_ = nullptr, *state_mean_ = nullptr, *state_std_ = nullptr,
          *action_mean_ = nullptr, *action_std_ = nullptr;
    // the cameras' normalized frames (with their block maxima
    // [n_cams][kConvPartMax] for an int8 stem), the trunk's features of every
    // camera
    float *norm_ = nullptr, *part_norm_ = nullptr, *feats_ = nullptr, *state_n_ = nullptr, *act_n_ = nullptr;
    hipStream_t own_ = nullptr;
    // The captured backbone graphs read the caller's frames in place (and the
    // encode graph writes the caller's features in place); a call with other
    // pointers starts a new capture under a new key.
    const uint8_t* pred_img_ = nullptr;
    const uint8_t* enc_img_ = nullptr;
    float* enc_feats_ = nullptr;
    uint64_t pred_key_ = 0, enc_key_ = 0;
    GraphReplay replay_, enc_replay_;
};

// ------------------------------------------------------------------ Octo --
// src/models/octo/octo_transformer.{h,cpp}: pre-LN ViT blocks over
// [task | per timestep: primary, wrist, (repeated task), readout] with the
// block-causal attends() rule, the final layer computed for the last readout
// row only. int8 mask bits as octo_model.cpp:60 (1 attention, 2 w1, 4 w2,
// 8 token projections). meta key repeat_task 0 drops the per-step task copy
// (the 16 + wnd * (256 + 64 + 1) token layout); the reference always repeats.
class OctoTf {
public:
    OctoTf(const std::string& dir, int int8_mask);
    ~OctoTf();
    int d() const { return d_; }
    int total_tokens(int wnd) const { return n_task_ + wnd * per_step(); }
    int readout_index(int wnd) const { return n_task_ + wnd * per_step() - 1; }
    int per_step() const { return tok_p_ + tok_w_ + (repeat_task_ ? n_task_ : 0) + n_readout_; }
    int max_horizon() const { return max_h_; }
    int n_task() const { return n_task_; }
    int tok_primary() const { return tok_p_; }
    int tok_wrist() const { return tok_w_; }
    int t5_dim() const { return t5_dim_; }
    int stem_dim() const { return stem_dim_; }
    int int8_layers() const { return n_int8_; }
    // device pointers; t5 [n_task, t5_dim], stem_p [wnd, tok_primary, stem_dim],
    // stem_w [wnd, tok_wrist, stem_dim] or null; timestep_mask host [wnd];
    // out [d] = the final-LayerNorm readout row.
    void forward_dev(const float* t5, const float* stem_p, const float* stem_w, int wnd,
                     const uint8_t* timestep_mask, float* out, hipStream_t caller);
    int graph_nodes() const { return replay_.nodes(); }

private:
    struct Layer {
        DLinear qkv, o, w1, w2;
        const float *ln1s, *ln1b, *ln2s, *ln2b;
    };
    void ensure(int wnd, const uint8_t* tmask, bool wrist);
    void run(hipStream_t st);

    int d_ = 384, n_layers_ = 12, heads_ = 6, hd_ = 64, mlp_ = 1536, max_h_ = 10, n_task_ = 16;
    int tok_p_ = 256, tok_w_ = 64, n_readout_ = 1, t5_dim_ = 768, stem_dim_ = 512;
    int repeat_task_ = 1, n_int8_ = 0;
    float eps_ = 1e-6f;
    bool gelu_erf_ = false;
    DeviceArena A_;
    DLinear proj_task_, proj_prim_, proj_wrist_;
    const float *pos_task_ = nullptr, *pos_prim_ = nullptr, *pos_wrist_ = nullptr,
                *pos_readout_ = nullptr, *final_s_ = nullptr, *final_b_ = nullptr;
    std::vector<Layer> layers_;
    // per-shape state: layout_ is (wnd, wrist, timestep mask) the buffers and
    // tables were built for, key_ counts layouts (the graph replay key)
    std::vector<uint8_t> layout_;
    uint64_t key_ = 0;
    int wnd_ = 0, total_ = 0, n_groups_ = 0;
    bool wrist_ = false;
    std::unique_ptr<DeviceArena> S_;
    float *t5_ = nullptr, *sp_ = nullptr, *sw_ = nullptr, *out_ = nullptr, *x_ = nullptr, *P_ = nullptr,
          *h_ = nullptr, *qkv_ = nullptr, *att_ = nullptr, *ff_buf_ = nullptr;
    uint8_t *qg_ = nullptr, *allow_ = nullptr;
    Ctx ctx_;
    hipStream_t own_ = nullptr;
    GraphReplay replay_;
};

// --------------------------------------------------------------- SmolVLA --
// src/models/smolvla/{smollm2_lm,action_expert,smolvla_model}.cpp: the SmolLM2
// prefix tower (RMSNorm, GQA with RoPE-NeoX, SwiGLU; K/V cached per layer)
// over the assembled prefix embeddings, then the action expert's flow-matching
// denoise (self-attention layers over prefix + suffix K/V, cross-attention
// layers over the re-projected prefix K/V) for num_steps Euler steps. int8
// mask bits as smolvla_model.cpp:44 (16 the text tower, 32 the expert).
class SmolvlaTf {
public:
    SmolvlaTf(const std::string& dir, int int8_mask);
    ~SmolvlaTf();
    int chunk() const { return C_; }
    int max_action_dim() const { return mad_; }
    int hidden() const { return H_; }
    int num_steps() const { return steps_; }
    int int8_layers() const { return n_int8_; }
    // device pointers; prefix [n_prefix, hidden] (scaled image/text embeddings
    // + the state token, as smolvla_model.cpp:231-250 assembles them); pad host
    // [n_prefix] (1 real, 0 padding; the last token is the state token);
    // noise [chunk, max_action_dim]; actions [chunk, max_action_dim] normalized.
    // Real-time chunking guidance (action_expert.cpp:377-389): guide
    // [chunk, max_action_dim] (the normalized previous chunk, zero past its
    // rows) and weights [chunk] on the device, the guidance weight of step s
    // min((1 - tau) / tau * ((1 - tau)^2 + tau^2) / (1 - tau)^2, max_guidance).
    struct Rtc {
        const float* guide;
        const float* weights;
        float max_guidance;
    };
    void chunk_dev(const float* prefix, const int32_t* pad, int n_prefix, const float* noise,
                   float* actions, hipStream_t caller, const Rtc* rtc = nullptr);
    int graph_nodes() const { return rtc_ ? replay_rtc_.nodes() : replay_.nodes(); }

private:
    struct VlmLayer {
        DLinear qkv, o, gu, down;
        const float *ln_in, *ln_post;
    };
    struct ExpLayer {
        bool self;
        DLinear q_or_qkv, k, v, o, gu, down;  // self: q_or_qkv = q|k|v; cross: q, k, v apart
        const float *ln_in, *ln_post;
    };
    void ensure(const int32_t* pad, int n_prefix);
    void run(hipStream_t st);

    // text tower
    int H_ = 960, nq_ = 15, nkv_ = 5, hd_ = 64, F_ = 2560, NL_ = 32;
    float eps_ = 1e-5f, rope_base_ = 10000.0f;
    // expert
    int EH_ = 480, EF_ = 1280, ENL_ = 32, enq_ = 15, enkv_ = 5, ehd_ = 64, san_ = 2, C_ = 50,
        steps_ = 10, mad_ = 32;
    float eeps_ = 1e-5f, erope_ = 10000.0f;
    double min_period_ = 4e-3, max_period_ = 4.0;
    int n_int8_ = 0;
    DeviceArena A_;
    std::vector<VlmLayer> vlm_;
    std::vector<ExpLayer> exp_;
    const float* out_norm_ = nullptr;
    DLinear ain_, at1_, at2_, aout_;
    // per-shape state: pad_ is the pad vector the buffers, masks and RoPE
    // tables were built for, key_ counts layouts (the graph replay key)
    std::vector<int32_t> pad_;
    uint64_t key_ = 0;
    int np_ = 0, SK_ = 0, QKVW_ = 0;
    std::unique_ptr<DeviceArena> S_;
    float *prefix_in_ = nullptr, *noise_in_ = nullptr, *act_out_ = nullptr, *h_ = nullptr,
          *xn_ = nullptr, *att_ = nullptr, *gu_raw_ = nullptr, *gu_ = nullptr, *eh_ = nullptr,
          *ehn_ = nullptr, *eq_ = nullptr, *mlp1_ = nullptr, *x_ = nullptr, *hf_ = nullptr;
    // guidance: the velocity, the guide, its row weights, the per-step weights
    float *v_ = nullptr, *guide_ = nullptr, *gweights_ = nullptr, *gw_ = nullptr;
    std::vector<float> gw_host_;
    bool rtc_ = false;
    std::vector<float*> qkv_;        // per text layer [np + C, QKVW]: prefix rows from the tower, suffix rows from the expert
    std::vector<float*> ck_, cv_;    // per cross layer [np, kv_full]
    std::vector<float*> at_;         // per step [C, 2 EH], right half = the step's time embedding
    double *rope_p_ = nullptr, *rope_full_ = nullptr, *rope_reb_ = nullptr;  // cos/sin tables
    uint8_t *pgroup_ = nullptr, *pallow_ = nullptr;
    float *dmask_ = nullptr, *cmask_ = nullptr;
    bool dcausal_ = true, cnone_ = true;
    Ctx ctx_;
    hipStream_t own_ = nullptr;
    // the plain and the guided denoise loops are different graphs; each keeps
    // its own, so alternating modes replay both
    GraphReplay replay_, replay_rtc_;
};

// ---------------------------------------------------------------- SigLIP --
// src/models/smolvla/siglip_vision.{h,cpp}: SmolVLA's vision tower (patch
// embedding + positions, n_layers pre-LN encoder layers with GELU tanh and
// full attention, post-LayerNorm) and its connector (pixel shuffle by
// scale_factor, bias-free modality projection). int8 mask bits as
// SmolvlaModel::apply_int8 (smolvla_model.cpp:127-140): 1 attention, 2 w1,
// 4 w2, 8 patch embedding + modality projection.
class SiglipTf {
public:
    SiglipTf(const std::string& dir, int int8_mask);
    ~SiglipTf();
    int img() const { return img_; }
    int n_tokens() const { return ntok_; }
    int out_dim() const { return mm_out_; }
    int hidden() const { return H_; }
    int int8_layers() const { return n_int8_; }
    // device pointers; pixels [3, img, img] (CHW, the preprocessed image),
    // out [n_tokens, out_dim] the image tokens before SmolVLA's sqrt(hidden)
    void encode_dev(const float* pixels, float* out, hipStream_t caller);
    int graph_nodes() const { return replay_.nodes(); }

private:
    struct Layer {
        DLinear qkv, o, w1, w2;
        const float *ln1s, *ln1b, *ln2s, *ln2b;
    };
    void run(hipStream_t st);

    int H_ = 768, heads_ = 12, hd_ = 64, I_ = 3072, NL_ = 12, P_ = 16, img_ = 512, NP_ = 1024, sf_ = 4,
        mm_out_ = 960, ntok_ = 64, side_ = 32, n_int8_ = 0;
    float eps_ = 1e-6f;
    DeviceArena A_;
    DLinear patch_, mm_;
    const float *pos_ = nullptr, *post_s_ = nullptr, *post_b_ = nullptr;
    std::vector<Layer> layers_;
    float *patches_ = nullptr, *x_ = nullptr, *h_ = nullptr, *qkv_ = nullptr, *att_ = nullptr, *ff_ = nullptr,
          *shuf_ = nullptr, *out_ = nullptr;
    Ctx ctx_;
    hipStream_t own_ = nullptr;
    GraphReplay replay_;
};

// ---------------------------------------------------- SmolVLA policy --
// src/models/smolvla/smolvla_model.{h,cpp} + smolvla_capi.cpp: native-size
// uint8 frames -> resize_with_pad -> SigLIP per view, the language tokens'
// bf16 embeddings, the projected normalized state -> the prefix -> SmolvlaTf
// (optionally with real-time-chunking guidance) -> un-normalized actions.
// Files: heads.meta, emb.bin, heads.bin, stats_{state,action}_{mean,std}.bin,
// config.txt (tokenizer_max_length, pad_token_id), vit.*, vlm.*, aex.*, and the
// tokenizer's vocab.txt + merges.txt in tok_dir. SMOLVLA_INT8 is read at load.
class SmolvlaModel {
public:
    SmolvlaModel(const std::string& dir, const std::string& tok_dir);
    ~SmolvlaModel();
    int chunk() const { return tf_->chunk(); }
    int action_dim() const { return real_action_dim_; }
    int state_dim() const { return real_state_dim_; }
    int max_action_dim() const { return tf_->max_action_dim(); }
    int n_views() const { return n_views_; }
    int img_size() const { return vit_->img(); }
    int tok_maxlen() const { return tok_maxlen_; }
    int int8_layers() const { return vit_->int8_layers() + tf_->int8_layers(); }
    int graph_nodes() const { return vit_->graph_nodes() + tf_->graph_nodes(); }
    // vla_smolvla_tokenize: ids / mask [tok_maxlen]; returns the token count
    int tokenize(const std::string& text, int32_t* ids, int32_t* mask) const;
    // host buffers as vla_smolvla_predict_rtc takes them; prev null or n_prev
    // 0 for no guidance. ShapeError for a token id outside the vocabulary.
    void predict(const uint8_t* frames, int nv, int height, int width, const int32_t* tokens,
                 const int32_t* lang_mask, int n_lang, const float* state, const float* noise, uint64_t seed,
                 float* actions, const float* prev, int n_prev, const float* weights, float max_guidance);
    // the preprocessed views [nv, 3, img, img] (host), for tests
    void preprocess(const uint8_t* frames, int nv, int height, int width, float* pixels);

private:
    void stage_frames(const uint8_t* frames, int nv, int height, int width);

    std::unique_ptr<SiglipTf> vit_;
    std::unique_ptr<SmolvlaTf> tf_;
    std::unique_ptr<BpeTokenizer> tok_;
    int tok_maxlen_ = 48, pad_id_ = 2;
    int vocab_ = 0, hidden_ = 0, max_state_dim_ = 0, real_state_dim_ = 0, real_action_dim_ = 0, n_views_ = 0;
    float norm_eps_ = 0.0f;
    DeviceArena A_;
    uint16_t* emb_ = nullptr;
    float *state_w_ = nullptr, *state_b_ = nullptr, *state_mean_ = nullptr, *state_std_ = nullptr,
          *action_mean_ = nullptr, *action_std_ = nullptr;
    float *pixels_ = nullptr, *state_raw_ = nullptr, *state_n_ = nullptr, *noise_ = nullptr, *act_n_ = nullptr,
          *actions_ = nullptr, *guide_ = nullptr, *prev_ = nullptr, *weights_ = nullptr;
    // per-call sizes: frames (native resolution) and the prefix (language length)
    std::unique_ptr<DeviceArena> F_, P_;
    size_t frames_cap_ = 0;
    int prefix_cap_ = -1;
    uint8_t* frames_ = nullptr;
    float* prefix_ = nullptr;
    int32_t* ids_ = nullptr;
    hipStream_t own_ = nullptr;
};

// ------------------------------------------------------------ Octo policy --

// src/nn/t5_encoder.{h,cpp}: the T5 encoder (pre-RMSNorm blocks, relative
// position bias attention without 1/sqrt(d) scaling, ReLU FFN, no biases,
// final RMSNorm), fp32 on the device. <stem>.meta / <stem>.bin.
class T5Enc {
public:
    // <stem>.meta / <stem>.bin. With tail set, the .bin may hold more floats
    // past the encoder (IMPACT's text heads, t5_text.cpp:41-64): they are
    // copied into *tail instead of failing the size check.
    T5Enc(const CkptFiles& files, const std::string& stem, std::vector<float>* tail = nullptr);
    int d_model() const { return D_; }
    int vocab() const { return vocab_; }
    // ids / mask host [seq] -> out device [seq, d_model]; an id outside the
    // vocabulary embeds as zeros (t5_encoder.cpp:96-104)
    void encode_dev(const int32_t* ids, const int32_t* mask, int seq, float* out, hipStream_t st);

private:
    struct Layer {
        const float *ln1, *ln2;
        float *wqkv, *wo, *wi, *wo2;
    };
    int D_ = 768, NL_ = 12, NH_ = 12, HD_ = 64, FF_ = 3072, vocab_ = 32128, nb_ = 32, maxd_ = 128;
    float eps_ = 1e-6f;
    DeviceArena A_;
    const float *emb_ = nullptr, *final_ = nullptr;
    std::vector<float> rel_;  // [n_buckets, n_heads] (host: the bias table is built per mask)
    std::vector<Layer> layers_;
    std::unique_ptr<DeviceArena> S_;
    int seq_cap_ = 0;
    float *x_ = nullptr, *h_ = nullptr, *qkv_ = nullptr, *att_ = nullptr, *ff_ = nullptr, *bias_ = nullptr;
    int32_t* ids_ = nullptr;
};

// src/models/octo/small_stem.{h,cpp}: uint8 RGB -> [x / 127.5 - 1, three -1
// goal channels] -> n_layers x (k x k conv, stride, pad -> GroupNorm + ReLU)
// -> patch embedding. int8_mask: OCTO_INT8 bit 16 the convs (conv2d_i8),
// bit 8 the embedding.
class OctoStem {
public:
    OctoStem(const CkptFiles& files, const std::string& name, int int8_mask, int H, int W);
    int tokens() const { return tok_; }
    int embed_dim() const { return embed_dim_; }
    int int8_layers() const { return n_int8_; }
    // img device [H, W, 3] uint8 -> out device [tokens, embed_dim]
    void encode_dev(const uint8_t* img, float* out, hipStream_t st);

private:
    struct Layer {
        int cin, cout, H, W, Ho, Wo;
        float *W_ = nullptr, *b = nullptr;
        const float *gs = nullptr, *gb = nullptr;
        std::unique_ptr<vla_linear_i8> q8;
    };
    int H_ = 0, W_ = 0, k_ = 3, stride_ = 2, pad_ = 1, groups_ = 32, embed_dim_ = 512, tok_ = 0, n_int8_ = 0;
    float gn_eps_ = 1e-6f;
    DeviceArena A_;
    std::vector<Layer> layers_;
    DLinear embed_;
    float *a_ = nullptr, *b_ = nullptr, *col_ = nullptr, *gA_ = nullptr, *gB_ = nullptr;
    size_t col_floats_ = 0;  // im2col rows + split-K sums
    double* gW_ = nullptr;   // GroupNorm partial sums
    size_t gw_doubles_ = 0;
    void* work_ = nullptr;
    size_t work_bytes_ = 0;
    Ctx ctx_;
};

// src/models/octo/diffusion_head.{h,cpp} + src/nn/diffusion.{h,cpp}: the DDPM
// score network on [time conditioning, readout embedding, x] and the
// `steps`-step reverse loop with clipping. int8_mask: OCTO_INT8 bit 32
// (in/out projections and the blocks' linears whose N % 16 == 0).
class OctoHead {
public:
    OctoHead(const CkptFiles& files, int int8_mask);
    int flat() const { return ad_ * horizon_; }
    int action_dim() const { return ad_; }
    int horizon() const { return horizon_; }
    int steps() const { return steps_; }
    int emb() const { return emb_; }
    int int8_layers() const { return n_int8_; }
    // device: emb [emb], noise [flat], z [steps, flat] -> actions [flat]
    void denoise_dev(const float* emb, const float* noise, const float* z, float* actions, hipStream_t st);

private:
    struct Block {
        const float *ln_s, *ln_b;
        DLinear d0, d1;
    };
    int emb_ = 384, ad_ = 7, horizon_ = 4, td_ = 32, nb_ = 3, H_ = 256, steps_ = 20, n_int8_ = 0;
    float max_action_ = 5.0f;
    DeviceArena A_;
    DLinear in_proj_, out_proj_;
    std::vector<Block> blocks_;
    float* cond_ = nullptr;  // [steps, time_dim], built at load
    std::vector<float> a1_, a2_, sb_;
    float *in_ = nullptr, *h_ = nullptr, *n_ = nullptr, *wide_ = nullptr, *e_ = nullptr;
    Ctx ctx_;
    OctoHeadArgs fused_;  // the one-workgroup form of denoise_dev
    bool fused_ok_ = false;
};

// src/models/octo/octo_model.{h,cpp} + octo_capi.cpp: pre-resized uint8
// frames (primary 256 x 256, wrist 128 x 128) -> SmallStems (a frame seen in
// this or the previous window reuses its tokens) -> OctoTf with the T5
// embedding of the instruction (cached per instruction) -> the readout ->
// DDPM head -> optional un-normalization. OCTO_INT8 is read at load.
class OctoModel {
public:
    OctoModel(const std::string& dir, const std::string& tok_dir);
    ~OctoModel();
    int horizon() const { return head_->horizon(); }
    int action_dim() const { return head_->action_dim(); }
    int max_window() const { return tf_->max_horizon(); }
    int int8_layers() const {
        return tf_->int8_layers() + sp_->int8_layers() + sw_->int8_layers() + head_->int8_layers();
    }
    // host pointers as vla_octo_predict_ex takes them
    void predict(const uint8_t* primary, const uint8_t* wrist, int wnd, const uint8_t* tmask,
                 const std::string& instruction, const float* noise, const float* z, uint64_t seed,
                 bool unnormalize, float* actions);
    // the T5 embedding of an instruction [n_task, t5_dim] (host), for tests
    void lang(const std::string& instruction, float* out);
    int64_t lang_size() const { return (int64_t)tf_->n_task() * t5_->d_model(); }

private:
    const float* lang_dev(const std::string& instruction);

    UnigramTokenizer tok_;
    std::unique_ptr<T5Enc> t5_;
    std::unique_ptr<OctoStem> sp_, sw_;
    std::unique_ptr<OctoTf> tf_;
    std::unique_ptr<OctoHead> head_;
    DeviceArena A_;
    float *act_mean_ = nullptr, *act_std_ = nullptr;
    // the instruction cache (octo_model.cpp:143-158): at most 64 entries
    std::map<std::string, std::unique_ptr<DeviceArena>> lang_arena_;
    std::map<std::string, const float*> lang_;
    // frames and stem tokens of this window and the previous one
    uint8_t *frames_p_ = nullptr, *frames_w_ = nullptr;
    float *tok_p_[2] = {nullptr, nullptr}, *tok_w_[2] = {nullptr, nullptr};
    int cur_ = 0;
    std::vector<uint8_t> prev_p_, prev_w_;
    float *emb_ = nullptr, *noise_ = nullptr, *z_ = nullptr, *act_ = nullptr, *out_ = nullptr;
    hipStream_t own_ = nullptr;
};

// ---------------------------------------------------------------- IMPACT --
// src/models/impact/{impact_model,t5_text}.{h,cpp}: ActModel with the IMPACT
// spec (FiLM points in the trunk, a text tail in the transformer; files
// config.txt, vision.meta/.bin, impact.meta/.bin, stats.bin) and a language
// pathway run once per instruction: the SentencePiece tokenizer (vocab.txt),
// the pruned-vocabulary remap (vocab_map.bin, config.txt's vocab_full and
// unk_id), T5-small (text.meta / .bin) and, from the tail of text.bin, the
// text projection, the learned text positions and the FiLM head. IMPACT_INT8
// (and IMPACT_I8_CONV_FROM / _TO) are read at load.
class ImpactModel {
public:
    explicit ImpactModel(const std::string& dir);
    ~ImpactModel();
    int chunk() const { return act_->chunk(); }
    int action_dim() const { return act_->action_dim(); }
    int state_dim() const { return act_->state_dim(); }
    int n_cams() const { return act_->n_cams(); }
    int img_h() const { return act_->img_h(); }
    int img_w() const { return act_->img_w(); }
    int n_text() const { return n_text_; }
    int film_total() const { return film_total_; }
    int int8_layers() const { return act_->int8_layers(); }
    int int8_convs() const { return act_->int8_convs(); }
    // tokenize, remap and encode an instruction; a no-op when it is the cached one
    void set_instruction(const std::string& instruction);
    bool have_text() const { return have_text_; }
    // device pointers: frames [n_cams, img_h, img_w, 3] uint8, state
    // [state_dim] raw, actions [chunk, action_dim]; the instruction set first
    void predict_dev(const uint8_t* frames, const float* state, bool unnormalize, float* actions,
                     hipStream_t caller);
    // the current instruction's language-side values (vla_impact_tokens / _film)
    const std::vector<int32_t>& token_ids() const { return ids_; }
    const std::vector<int32_t>& compact_ids() const { return compact_; }
    const std::vector<int32_t>& token_mask() const { return mask_; }
    const std::vector<float>& film_gamma() const { return gamma_; }
    const std::vector<float>& film_beta() const { return beta_; }

private:
    int remap(const std::vector<int32_t>& ids, std::vector<int32_t>& compact);

    std::unique_ptr<ActModel> act_;
    UnigramTokenizer tok_;
    std::unique_ptr<T5Enc> t5_;
    DeviceArena A_;
    int proj_dim_ = 512, n_text_ = 32, film_total_ = 960, vocab_full_ = 32128, unk_id_ = 2, unk_compact_ = 0;
    std::vector<int32_t> vocab_map_;
    float *proj_w_ = nullptr, *proj_b_ = nullptr, *text_pos_ = nullptr, *film_w_ = nullptr, *film_bias_ = nullptr;
    float *h_ = nullptr, *text_tok_ = nullptr, *pooled_ = nullptr, *gb_ = nullptr;
    int32_t* mask_d_ = nullptr;
    bool have_text_ = false, warned_oov_ = false;
    std::string cached_;
    std::vector<int32_t> ids_, compact_, mask_;
    int n_real_ = 0;
    std::vector<float> gamma_, beta_;
    hipStream_t own_ = nullptr;
};

// ------------------------------------------------------- Diffusion Policy --
// src/models/diffusion/{diffusion_model,unet1d,rgb_encoder,scheduler}.{h,cpp}:
// n_obs_steps frames per camera and n_obs_steps states in, the executed slice
// of the denoised horizon out. Per camera a GroupNorm ResNet-18 trunk, a 1x1
// conv to keypoints, the spatial soft-argmax and a Linear + ReLU give 2 K
// features per frame (frames seen by the previous query are not encoded
// again, as the reference's pixel cache does); the conditional 1-D UNet
// (Conv1d + GroupNorm + Mish blocks with FiLM from [time embedding | global
// conditioning], strided-conv downsampling, transposed-conv upsampling with
// skip concatenation) runs once per DDPM / DDIM step. Files: diffusion.meta,
// rgb_encoder<i>_backbone.meta/.bin, rgb_encoder<i>.bin, unet.bin, stats.bin.
// DIFFUSION_INT8 (read at load as diffusion_model.cpp:111-119): bit 1 the
// UNet's conv / residual / downsample GEMMs, bit 2 every encoder conv;
// DP_STEPS and DP_SCHEDULER override the checkpoint's sampler.
//
// On the device the UNet's convolutions are GEMMs over "taps views": each
// activation [T, C] sits between zero rows, so output row t of a k-tap,
// stride-s convolution reads the k * C consecutive floats from row t * s -
// pad, i.e. the sequence itself with row stride s * C (rows overlap); the
// transposed convolution is two such GEMMs (even and odd output rows). The
// FiLM vectors of every block and every step are one GEMM per query, since
// the step's half of each block's conditioning input does not depend on the
// observation. The whole sampler loop is one HIP graph.
class DiffusionModel {
public:
    explicit DiffusionModel(const std::string& dir);
    ~DiffusionModel();
    int chunk() const { return n_action_; }
    int horizon() const { return H_; }
    int action_dim() const { return A_dim_; }
    int state_dim() const { return sd_; }
    int n_cams() const { return n_cams_; }
    int n_obs() const { return n_obs_; }
    int img_h() const { return img_h_; }
    int img_w() const { return img_w_; }
    int num_steps() const { return (int)timesteps_.size(); }
    bool is_ddim() const { return ddim_; }
    int int8_layers() const { return n_int8_; }
    int int8_convs() const;
    int graph_nodes() const { return replay_.nodes(); }
    // host pointers: frames [n_obs, n_cams, img_h, img_w, 3] uint8 oldest
    // first, state [n_obs, state_dim] raw, noise [1 + num_steps, horizon,
    // action_dim] or null (start from zeros, no DDPM noise), actions
    // [chunk, action_dim]
    void predict(const uint8_t* frames, const float* state, const float* noise, bool unnormalize, float* actions);

private:
    struct Act {  // [T, C] rows at p, with P zero rows before and after
        float* p = nullptr;
        int T = 0, C = 0;
    };
    struct ConvB {  // Conv1d (taps GEMM) -> GroupNorm -> Mish
        DLinear L;
        int cin = 0, cout = 0;
        const float *gs = nullptr, *gb = nullptr;
    };
    struct Res {
        ConvB c1, c2;
        DLinear res;  // 1x1 conv when cin != cout
        bool has_res = false;
        int cin = 0, cout = 0, film_off = 0;
        Act h, o;
        float* rb = nullptr;    // the 1x1 conv's output, added by the second norm
        float* out2 = nullptr;  // a second home of o: its place in a later concatenation
        int ldo2 = 0;
    };
    struct Down {
        Res r1, r2;
        DLinear ds;
        bool has = false;
        Act out;  // the downsampled sequence
    };
    struct Up {
        Res r1, r2;
        DLinear even, odd;  // the transposed conv's even / odd output rows
        bool has = false;
        int uc = 0;
        Act cat, out;
        float* up_to = nullptr;  // where the transposed conv writes: the next cat, or out
        int up_ld = 0;
    };
    struct Encoder {
        std::unique_ptr<ResNetTrunk> trunk;
        DLinear kp, out;
        float* grid = nullptr;  // [fh * fw, 2]
    };
    Act act(int T, int C);
    void conv(const Ctx& c, const DLinear& L, const Act& x, int k, int stride, float* out, int ldo, int rows) const;
    void res_block(const Ctx& c, const Res& r, const Act& x, int step) const;
    void unet(const Ctx& c, int step) const;
    void sample(hipStream_t st);
    void encode(int slot, hipStream_t st);

    // diffusion.meta
    int n_obs_ = 2, n_cams_ = 2, img_h_ = 480, img_w_ = 640, crop_h_ = 0, crop_w_ = 0, sd_ = 6, A_dim_ = 6, H_ = 64,
        n_action_ = 32, kp_ = 32, k_ = 5, groups_ = 8, D_ = 128, n_train_ = 100, n_infer_ = 100;
    std::vector<int> down_dims_;
    bool film_scale_ = true, clip_ = true, separate_ = true, ddim_ = false;
    float clip_range_ = 1.0f, gn_eps_ = 1e-5f;
    int P_ = 2, CD_ = 0, G_ = 0, F_ = 0, n_int8_ = 0, n_cond_ = 0, top_ = 0, left_ = 0, oh_ = 0, ow_ = 0;
    // the sampler: alphas_cumprod and the descending timestep ladder
    std::vector<double> alphas_cumprod_;
    std::vector<int> timesteps_;
    DeviceArena Ad_;
    Ctx ctx_;
    std::vector<Encoder> enc_;
    DLinear cond_;  // every block's cond encoder, rows concatenated
    std::vector<Down> down_;
    Res mid1_, mid2_;
    std::vector<Up> up_;
    ConvB final_;
    DLinear final_conv_;
    float *smin_ = nullptr, *smax_ = nullptr, *amin_ = nullptr, *amax_ = nullptr, *img_mean_ = nullptr,
          *img_std_ = nullptr;
    // per query: frames and features per (step, camera) slot, the state rows,
    // the noise, the conditioning rows, the FiLM vectors of every step
    uint8_t* frames_ = nullptr;
    float *norm_ = nullptr, *fmap_ = nullptr, *kpmap_ = nullptr, *kpts_ = nullptr, *feats_ = nullptr,
          *state_ = nullptr, *noise_ = nullptr, *gcond_ = nullptr, *temb_ = nullptr, *gm_ = nullptr,
          *cond_all_ = nullptr, *eps_ = nullptr, *act_out_ = nullptr;
    Act x0_, f_;
    std::vector<std::vector<uint8_t>> slot_px_;  // the frame each slot last encoded (host)
    std::vector<std::unique_ptr<GraphReplay>> enc_replay_;
    hipStream_t own_ = nullptr;
    GraphReplay replay_;
};

}  // namespace hip
}  // namespace vla
