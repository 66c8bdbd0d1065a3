// common.h - shared plumbing of the gfx950 backend: error types that the C ABI
// maps to vla_status, HIP call checking, and small device helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

namespace vla {
namespace hip {

// A HIP runtime failure. The C ABI turns it into VLA_ERR_EXCEPTION.
struct HipError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// A precondition the reference asserts (or an out-of-range argument). The C ABI
// turns it into VLA_ERR_ARG.
struct ArgError : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};

// An input whose shape or content the model cannot take (the reference's
// VLA_ERR_SHAPE, include/vla_simd.h:46-51).
struct ShapeError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

[[noreturn]] void throw_hip(hipError_t e, const char* what, const char* file, int line);

#define VLA_HIP_CHECK(expr)                                                    \
    do {                                                                       \
        hipError_t vla_e_ = (expr);                                            \
        if (vla_e_ != hipSuccess) ::vla::hip::throw_hip(vla_e_, #expr, __FILE__, __LINE__); \
    } while (0)

#define VLA_LAUNCH_CHECK() VLA_HIP_CHECK(hipGetLastError())

#define VLA_REQUIRE(cond, msg)                                                 \
    do {                                                                       \
        if (!(cond)) throw ::vla::hip::ArgError(msg);                          \
    } while (0)

inline int kpad4(int K) { return (K + 3) & ~3; }
inline int round_up(int v, int m) { return (v + m - 1) / m * m; }
inline bool aligned(const void* p, size_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// int8 K bound of nn::Linear::init_int8 (src/nn/linear.cpp:67): the x86
// kernel's unsigned-biased accumulator must stay in int32. The GPU one is
// signed (|acc| <= K*127*127) but keeps the same bound so the two backends
// accept the same layers.
constexpr int kMaxI8K = 2147483647 / (255 * 127);

// Fixed widths of the device code.
constexpr int kWave = 64;

// ---- kernel launchers (defined in the .hip files) ----

// quant.hip
// the same quantization written in the panel layout (rows <= kPanelMaxRows),
// panel_bytes(rows, K) bytes at xq
// taps: the rows of x may overlap (ldx < K), a view that reads a 1-D
// convolution's taps straight from the padded sequence (x is only read)
void launch_quantize_rows_panel(const float* x, int ldx, int8_t* xq, float* scale, int rows, int K,
                                hipStream_t st, bool taps = false);
void launch_quantize_rows(const float* x, int ldx, int8_t* xq, int ldq, float* scale,
                          int rows, int K, hipStream_t st, bool taps = false);
// q[i] = clamp(rne(x[i] * inv), +-127) over n elements (quantize_span_i8)
void launch_quantize_span(const float* x, int8_t* q, int64_t n, float inv, hipStream_t st);

// gemm_i8.hip: epilogue selects raw int32 output (acc32 != nullptr) or the
// fused dequant/bias/act(/accumulate) fp32 store.
// Panel layout of quantized activations (M <= 128, the skinny GEMM's input):
// K is cut into 64-byte panels, each holding every row's 64 bytes back to
// back over round_up(M, 16) rows, so element (m, k) sits at byte
// (k / 64) * panel_rows(M) * 64 + m * 64 + k % 64. One MFMA fragment (16 rows x
// 64 bytes) is then 1 KiB of contiguous memory, which one wave load reads as
// whole cache lines; row-major rows would cost 16 half-lines per load.
// Bytes [K, round_up(K, 64)) of every row are zero; rows [M, panel_rows(M))
// are never read into a stored output.
__host__ __device__ inline int panel_rows(int M) { return (M + 15) & ~15; }
inline size_t panel_bytes(int M, int K) { return (size_t)panel_rows(M) * (size_t)((K + 63) & ~63); }
constexpr int kPanelMaxRows = 128;

struct GemmArgs {
    const int8_t* A;  int lda;   // quantized activations [M, lda] (row-major; unused when a_panel)
    const int8_t* B;  int ldb;   // int8 weights [N, ldb]
    const float* ascale;         // [M]
    const float* wscale;         // [N]
    const float* bias;           // [N] or null
    float* out;       int ldo;   // [M, ldo]
    int32_t* acc32;              // raw accumulators [M, N] (test path) or null
    int M, N, K;
    int act;                     // vla_act
    int accumulate;              // out += result
    int a_panel;                 // A in the panel layout above (M <= kPanelMaxRows)
    // Split-K workspace (device, 16-byte aligned) or null. With it, a GEMM
    // whose tiles would leave most CUs idle and whose K is long runs as
    // gemm_split_plan's S partial products over K chunks (raw int32 sums into
    // the workspace) plus one reduce + epilogue pass; int32 sums are exact, so
    // the values are the same as without it.
    int32_t* split_ws;
    size_t split_bytes;
    int kchunk;                  // set by launch_gemm_i8 for a split launch
    // Rotating epilogue (the skinny GEMM only, M <= 128): output columns
    // [0, rope_cols) are heads of rope_hd columns, rotated after the epilogue
    // with the per-row table rope_cs [M][rope_hd / 2][cos, sin] (double), as
    // launch_rope_table would rotate them in place afterwards; null: none.
    const double* rope_cs;
    int rope_cols, rope_hd;
    // Convolution epilogue (launch_gemm_i8_conv only): with resid, out =
    // relu_gt(v + resid[m][n]) (stride ldo), the residual add + ReLU of a
    // ResNet block; without it act must be 1 (ReLU). omax receives each
    // block's max |out|, the block maxima the next conv2d_i8 folds into its
    // scale.
    const float* resid;
    float* omax;
    // Implicit convolution A (launch_gemm_i8_conv_implicit only): A is the
    // int8 NHWC map [cv_h, cv_w, cv_c] and row m of the product is output
    // pixel m of a cv_k x cv_k, stride cv_s, pad cv_p convolution (cv_wo
    // output columns), K = cv_k^2 cv_c in [ky][kx][ci] order, zero outside.
    int cv_h, cv_w, cv_c, cv_k, cv_s, cv_p, cv_wo;
};
void launch_gemm_i8(const GemmArgs& a, hipStream_t st);
// The product with the convolution epilogue above when the kernel
// launch_gemm_i8 would pick for the shape carries it (the unsplit skinny
// kernel, or the 32 x 64 x 128 LDS tile) and its maxima fit in 4096 floats:
// returns how many maxima it wrote. Returns 0, launching nothing, otherwise;
// the caller then runs launch_gemm_i8 and the separate ReLU pass.
int launch_gemm_i8_conv(const GemmArgs& a, hipStream_t st);
// The convolution as the 32 x 64 x 128 LDS GEMM tile gathering A from the
// int8 map (the cv_ fields; cv_c % 64 == 0, 16-byte aligned operands), with
// the convolution epilogue when omax is set. Returns the maxima written (0
// without omax).
int launch_gemm_i8_conv_implicit(const GemmArgs& a, hipStream_t st);
// The same with the skinny kernel (rows in the skinny GEMM's mid range,
// gemm_i8_conv_skinny_fits), its A fragments loaded straight from the map.
bool gemm_i8_conv_skinny_fits(int M, int N);
int launch_gemm_i8_conv_skinny_implicit(const GemmArgs& a, hipStream_t st);
// Two independent products over the same rows as one skinny launch (same
// bits as two launch_gemm_i8 calls). Returns false, launching nothing, when
// either would not take the unsplit skinny kernel; the caller then runs them
// one by one.
bool launch_gemm_i8_pair(const GemmArgs& a1, const GemmArgs& a2, hipStream_t st);
// Workspace bytes launch_gemm_i8 uses to split K for this shape (0: no split).
size_t gemm_split_bytes(int M, int N, int K);

// attn.hip
struct AttnArgs {
    float* out; int ldo;
    const float* Q; int ldq;
    const float* K; int ldk;
    const float* V; int ldv;
    int seq_q, seq_k, n_q, n_kv, head_dim;
    float scale;
    int mask_kind;
    const float* mask; int ldm;
    int causal_offset;
    int n_groups;
    const uint8_t* q_group;
    const uint8_t* k_group;
    const uint8_t* allow;
};
void launch_attention(const AttnArgs& a, hipStream_t st);

// eltwise.hip
void launch_layernorm(float* out, const float* x, const float* w, const float* b, int rows,
                      int hidden, float eps, hipStream_t st);
void launch_rmsnorm(float* out, const float* x, const float* w, int rows, int hidden, float eps,
                    hipStream_t st);
void launch_act(float* x, int64_t n, int act, hipStream_t st);
void launch_silu_gate(float* out, const float* g, const float* u, int64_t n, hipStream_t st);
void launch_add(float* out, const float* a, const float* b, int64_t n, hipStream_t st);
void launch_silu_gate_rows(float* out, int ldo, const float* g, int ldg, const float* u, int ldu,
                           int rows, int cols, hipStream_t st);
void launch_rope_neox(float* x, int ld, const int32_t* pos, int seq, int n_heads, int head_dim,
                      float base, hipStream_t st);
// Row kernels that end in the int8 quantizer (eltwise.hip). Per row, y is
// op 0 x itself, 1 LayerNorm(x; w, b), 2 RMSNorm(x; w), 3 silu_gate(x, u) (x
// the gate rows); then y goes to out (fp32, optional), to q/qs quantized (optional),
// and y + add (ACT's x + pos) to out2 / q2 / qs2 (each optional). The
// quantized bytes are those of launch_quantize_rows on the fp32 result.
struct RowQArgs {
    int op = 0;
    const float* x = nullptr;   int ldx = 0;
    const float* u = nullptr;   int ldu = 0;
    const float* w = nullptr;
    const float* b = nullptr;
    float eps = 0.0f;
    float* out = nullptr;       int ldo = 0;
    int8_t* q = nullptr;        int ldq = 0;  float* qs = nullptr;
    const float* add = nullptr; int ld_add = 0;
    float* out2 = nullptr;      int ldo2 = 0;
    int8_t* q2 = nullptr;       int ldq2 = 0; float* qs2 = nullptr;
    int rows = 0, H = 0;
    int q_panel = 0;            // q and q2 in the panel layout (ldq, ldq2 unused)
    int taps = 0;               // x rows may overlap (ldx < H; launch_gemm_i8_rowop only)
};
void launch_rowq(const RowQArgs& a, hipStream_t st);

// A skinny int8 GEMM that builds its own activations: every block applies the
// row op of `r` (op 0 identity, 2 RMSNorm or 3 silu_gate; no add, no fp32 out)
// to the fp32 rows, quantizes them per row into LDS (panel layout) exactly as
// launch_rowq would, and multiplies by g's int8 weights. g: B, ldb, wscale,
// bias, out, ldo, M (= r.rows), N, K (= r.H), act, accumulate (A, lda, ascale,
// acc32, a_panel unused); out must not overlap the rows read. rowop_gemm_fits
// says whether op and shape are supported (M <= 128, K % 4 == 0, K <= 2048,
// the panel within LDS).
bool rowop_gemm_fits(int op, int M, int K);
// Rows each block of the fused kernel applies the row op to (16 x FM: its row
// group of M for an output N columns wide).
int rowop_gemm_block_rows(int M, int N);
void launch_gemm_i8_rowop(const RowQArgs& r, const GemmArgs& g, hipStream_t st);

// conv.hip: conv2d_i8 (NHWC x [H, Wd, Cin] -> out [Hout, Wout, Cout]) as
// per-tensor quantize + im2col + the int8 GEMM. Weights Wq [Cout, ldw] over
// K = k*k*Cin (taps [ky][kx][ci]), per-channel wscale, optional bias. work:
// device scratch of at least conv_shape().work bytes, 256-byte aligned.
// clip <= 0 takes TCPU_I8_CLIP from the environment (default 1).
struct ConvShape {
    int Hout, Wout, npix, K, lda;
    size_t split;  // split-K workspace of the GEMM (gemm_split_bytes)
    size_t work;   // everything, split workspace last
};
ConvShape conv_shape(int H, int Wd, int Cin, int k, int stride, int pad, int Cout);
struct ConvArgs {
    float* out;
    const float* x;
    const int8_t* Wq;
    int ldw;
    const float* wscale;
    const float* bias;
    int H, Wd, Cin, Cout, k, stride, pad;
    float clip;
    void* work;
    size_t work_bytes;
    // optional: the block maxima of |x| its producer wrote (in_nparts <= 4096
    // floats, their max = max |x|); then no absmax pass over x runs
    const float* in_part = nullptr;
    int in_nparts = 0;
    // optional (a ResNet trunk's producer chain): out_part receives the block
    // maxima of |out| (at most 4096 floats) when the kernel taking the shape
    // fuses the epilogue that follows the conv - ReLU, or with resid ([npix,
    // Cout], 16-byte aligned) the residual add + ReLU (relu_gt(v + resid)).
    // The launcher then returns how many maxima it wrote; 0 means it ran the
    // plain conv, and the caller applies the ReLU pass itself.
    float* out_part = nullptr;
    const float* resid = nullptr;
    // optional (a ResNet downsample and the block's first conv, both over the
    // block input with the same output grid): xq_out is set to 1 when the
    // call left x's int8 map and its npix row scales in work (the LDS
    // implicit form), else 0; xq_in says work still holds them from the
    // previous call on the same x, maxima, workspace and output grid, so the
    // LDS implicit form skips its quantization pass (other forms ignore it).
    int* xq_out = nullptr;
    bool xq_in = false;
    // optional, with out_part (a stem followed by a max pool + ReLU): the
    // stored outputs stay as they are and out_part receives the block maxima
    // of max(0, out); only the word-per-pixel form does this (else 0 maxima)
    bool relu_maxima = false;
};
int launch_conv2d_i8(const ConvArgs& a, hipStream_t st);
// The max pool + ReLU of in_x [H, Wd, a.Cin] (window k, stride, pad) into
// a.x ([a.H, a.Wd, a.Cin], the conv a's input), which also leaves a.x's int8
// map and row scales in a.work for a with xq_in, the scale folded from
// a.in_part: the maxima of max(0, in_x) (relu_maxima). Returns 1, or 0
// (launching nothing) when a does not take a form that reads the map, the
// windows do not cover in_x or the operands do not fit.
int launch_conv_pool_quant(const ConvArgs& a, const float* in_x, int H, int Wd, int k, int stride, int pad,
                           hipStream_t st);
// Producers of a conv2d_i8 input that also write its block maxima (part:
// at most kConvPartMax floats per launch, per camera for the normalization;
// the launchers return how many) so the conv skips its absmax pass.
constexpr int kConvPartMax = 512;
// The most block maxima a conv2d_i8 folds, and so the most a fused conv
// epilogue may write (ConvArgs::out_part, GemmArgs::omax).
constexpr int kConvPartsFused = 4096;

// backbone.hip: ACT's image backbone around its GEMMs (NHWC fp32 maps)
// (pixel / 255 - mean[cam][c]) / (std[cam][c] + eps) for n_cams frames of npx pixels
int launch_normalize_u8(float* out, const uint8_t* img, int n_cams, int64_t npx, const float* mean,
                        const float* stdv, float eps, hipStream_t st, float* part = nullptr);
// col [Hout * Wout, ldc]: the k x k taps [ky][kx][ci] of every output pixel, zero outside
void launch_im2col_f32(float* col, int ldc, const float* x, int H, int Wd, int Cin, int k, int stride, int pad,
                       int Hout, int Wout, hipStream_t st);
// max pool with -inf padding, then the folded relu (!(v > 0) -> 0); part
// holds max_parts floats (at most kConvPartsFused)
int launch_maxpool_relu(float* out, const float* x, int H, int Wd, int C, int k, int stride, int pad, int Hout,
                        int Wout, hipStream_t st, float* part = nullptr, int max_parts = kConvPartMax);
// o = o + idn > 0 ? o + idn : 0
int launch_add_relu(float* o, const float* idn, int64_t n, hipStream_t st, float* part = nullptr);
// o = fma(1 + gamma[c], relu(o + idn), beta[c]) over NHWC maps of C channels
// (IMPACT's FiLM points); part as launch_add_relu, of |o|
int launch_add_relu_film(float* o, const float* idn, int64_t n, int C, const float* gamma, const float* beta,
                         hipStream_t st, float* part = nullptr);
// out[i] = (sum over the rows t with mask[t] != 0 of x[t][i], in row order) *
// (1 / live), i < D; zeros when no row is live (t5_text.cpp:115-128)
void launch_masked_row_mean(float* out, const float* x, int ldx, const int32_t* mask, int rows, int D,
                            hipStream_t st);
// x < 0 -> 0
int launch_relu_inplace(float* x, int64_t n, hipStream_t st, float* part = nullptr);
// [rows, cols] per column: mode 0 (x - a) / (b + eps), mode 1 fma(x, b, a)
void launch_col_affine(float* out, const float* x, int rows, int cols, const float* a, const float* b, float eps,
                       int mode, hipStream_t st);

// RoPE-NeoX from a cos/sin table cs[(t * head_dim/2 + i) * 2 + {0, 1}]
// (double; rope_cos_sin in graph.h builds it the way rope_neox does)
void launch_rope_table(float* x, int ld, const double* cs, int seq, int n_heads, int head_dim,
                       hipStream_t st);

// dst[r, c] = src[r, c] for a [rows, cols] block with row strides ldd / lds
void launch_copy_rows(float* dst, int ldd, const float* src, int lds, int rows, int cols,
                      hipStream_t st);

// vision.hip: SigLIP patch extraction, pixels [3, img, img] (CHW) ->
// out [(img/patch)^2, 3*patch^2] rows (ic, kh, kw) (conv.cpp:179-190), and the
// pixel shuffle of [side*side, hidden] patch rows into [(side/sf)^2,
// sf*sf*hidden] tokens (siglip_vision.cpp:188-198)
void launch_extract_patches(float* out, const float* pixels, int img, int patch, hipStream_t st);
void launch_pixel_shuffle(float* dst, const float* src, int side, int hidden, int sf, hipStream_t st);

// policy.hip: the model-level glue kernels.
// resize_with_pad (src/preprocess/image.cpp:13-51) of n_views uint8 HWC frames
// [h, w, 3] to CHW [3, S, S] canvases in [-1, 1], padding -1 at the top/left;
// resize_geometry is its host-side geometry (padding and source steps)
void resize_geometry(int h, int w, int S, int* pad_h, int* pad_w, double* sy, double* sx);
void launch_resize_with_pad(float* dst, const uint8_t* src, int n_views, int h, int w, int S, hipStream_t st);
// dst [n, H] = bf16 rows table[ids[t]] as fp32 * scale
void launch_embed_bf16(float* dst, const uint16_t* table, const int32_t* ids, int n, int H, float scale,
                       hipStream_t st);
void launch_scale(float* x, int64_t n, float s, hipStream_t st);
// out [rows, ldo]: (x[r, c] - mean[c]) / (std[c] + eps) for r < n_real, 0 for
// later rows; columns >= cols are not written
void launch_normalize_pad(float* out, int ldo, const float* x, int n_real, int rows, int cols, const float* mean,
                          const float* stdv, float eps, hipStream_t st);
// out [rows, cols] = fma(a[r, c], std[c] + eps, mean[c]) from a [rows, lda]
void launch_unnormalize(float* out, const float* a, int lda, int rows, int cols, const float* mean,
                        const float* stdv, float eps, hipStream_t st);
// dst [n, D] = fp32 rows table[ids[t]], zeros for ids outside [0, vocab)
void launch_embed_f32(float* dst, const float* table, const int32_t* ids, int n, int D, int vocab,
                      hipStream_t st);
// Octo SmallStem input: [npx, 6] = RGB / 127.5 - 1, then three -1 channels
void launch_stem_input(float* out, const uint8_t* img, int64_t npx, hipStream_t st);
// GroupNorm over NHWC [n_pixels, C <= 1024], groups of <= 256 channels, with per-channel scale / bias,
// then the optional ReLU; A / B: device scratch [C] each (the per-channel
// affine), work: groupnorm_work_doubles(n_pixels, C) doubles of partial sums
size_t groupnorm_work_doubles(int n_pixels, int C);
void launch_groupnorm(float* out, const float* x, const float* scale, const float* bias, int n_pixels, int C,
                      int groups, float eps, bool relu, float* A, float* B, double* work, size_t work_doubles,
                      hipStream_t st);
// out [steps, TD] = [cos(2 pi t w) | sin(2 pi t w)], t = 0..steps-1
void launch_fourier(float* out, const float* w, int steps, int TD, hipStream_t st);
void launch_concat3(float* out, const float* a, int na, const float* b, int nb, const float* c, int nc,
                    hipStream_t st);
// x = clip(a1 * (x - a2 * e) + sb * z, +-max_action) over n values
// Octo's DDPM head for all steps in one workgroup (policy.hip): one linear
// layer's weights, int8 (Wq [N, ldw] + ws + b) or fp32 (W [N, K] + b)
struct HeadLin {
    const int8_t* Wq = nullptr;
    const float* W = nullptr;
    const float* ws = nullptr;
    const float* b = nullptr;
    int ldw = 0, N = 0, K = 0;
};
constexpr int kOctoHeadMaxBlocks = 8;
struct OctoHeadArgs {
    HeadLin in_proj, out_proj, d0[kOctoHeadMaxBlocks], d1[kOctoHeadMaxBlocks];
    const float* ln_s[kOctoHeadMaxBlocks] = {};
    const float* ln_b[kOctoHeadMaxBlocks] = {};
    float ln_eps = 1e-6f;
    int nb = 0, H = 0, TD = 0, emb = 0, flat = 0, steps = 0;
    const float* cond = nullptr;   // [steps, TD]
    const float* embv = nullptr;   // [emb]
    const float* noise = nullptr;  // [flat]
    const float* z = nullptr;      // [steps, flat]
    const float* coef = nullptr;   // [steps][a1, a2, sb]
    float max_action = 0.0f;
    float* actions = nullptr;      // [flat]
};
// dynamic LDS of the fused head; launch_octo_head requires <= 64 KiB and
// 4 H, N <= 1024 outputs per layer
size_t octo_head_lds_bytes(int H, int TD, int emb, int flat);
void launch_octo_head(const OctoHeadArgs& a, hipStream_t st);
void launch_ddpm_step(float* x, const float* e, const float* z, int n, float a1, float a2, float sb,
                      float max_action, hipStream_t st);
// the guided Euler step of real-time chunking, gw [steps] on the device
void launch_rtc_step(float* x, const float* v, const float* prev, const float* weights, const float* gw, int step,
                     int rows, int cols, float time, float dt, hipStream_t st);

// diffusion.hip: Diffusion Policy's glue (models/diffusion/*.cpp).
// GroupNorm of [T, C] rows in `groups` groups (<= kDpGnMaxGroup channels
// each), then mish, then the FiLM fmaf(film_scale[c], y, film_bias[c]) or
// y + film_bias[c] (film_scale null), or the residual y + res[t, c];
// stored to out (which may be x) and, when given, out2 (row stride ldo2)
constexpr int kDpGnMaxGroup = 2048;
void launch_dp_gn_mish(float* out, int ldo, const float* x, int ldx, int T, int C, int groups, const float* scale,
                       const float* bias, float eps, const float* film_scale, const float* film_bias,
                       const float* res, int ldr, hipStream_t st, float* out2 = nullptr, int ldo2 = 0);
// out [C, 2]: per channel of x [npx, C], the softmax-weighted grid [npx, 2]
void launch_spatial_softmax(float* out, const float* x, const float* grid, int npx, int C, hipStream_t st);
// out [oh, ow, 3] = (img[top + y, left + x] / 255 - mean) / (std + eps) of an [H, W, 3] uint8 frame
void launch_crop_normalize(float* out, const uint8_t* img, int H, int W, int top, int left, int oh, int ow,
                           const float* mean, const float* stdv, float eps, hipStream_t st);
// g [steps, sd + n_cams F]: MIN_MAX-normalized state rows and the features
void launch_dp_gcond(float* g, const float* state, const float* smin, const float* smax, const float* feats,
                     int steps, int sd, int n_cams, int F, float eps, hipStream_t st);
// gm [steps, D + G] = [temb rows | mish(gcond)]
void launch_dp_cond_rows(float* gm, const float* temb, const float* gcond, int steps, int D, int G,
                         hipStream_t st);
void launch_mish(float* x, int64_t n, hipStream_t st);
// one DDPM (c0 x0 + c1 x + var z) or DDIM (c0 x0 + c1 e) step over n values
void launch_dp_sched_step(float* x, const float* e, const float* z, int n, double sqrt_ap, double sqrt_bp,
                          double c0, double c1, double var, bool ddim, bool clip, double range, hipStream_t st);
// out [chunk, A] = rows start.. of x [*, A], MIN_MAX un-normalized when unnorm
void launch_dp_actions(float* out, const float* x, int start, int chunk, int A, const float* amin,
                       const float* amax, float eps, bool unnorm, hipStream_t st);

// linear_f32.hip: out[m, n] = act(x[m,:] . W[n,:] + bias[n]); accumulate != 0
// adds it as fmaf(alpha, v, out[m, n]). act as vla_act, plus 4 = silu.
// out [Hout*Wout, Cout] = the k x k conv of the NHWC map x with W [Cout][k*k*Cin]
// (im2col's column order) as one implicit GEMM; false when the shape or
// alignment does not suit it (the caller then runs im2col + launch_linear_f32,
// which gives the same values)
bool launch_conv_f32_implicit(float* out, const float* x, int H, int Wd, int Cin, int k, int stride, int pad,
                              int Hout, int Wout, const float* W, const float* bias, int Cout, int act,
                              hipStream_t st, float* work = nullptr, size_t work_floats = 0);
// floats of npix im2col rows of K columns (rows padded to 4 floats), rounded up
// to 64 floats so what follows stays 256-byte aligned
inline size_t col_rows_floats(size_t npix, int K) { return (npix * (size_t)((K + 3) & ~3) + 63) / 64 * 64; }
// floats of the split-K workspace launch_linear_f32 (and the implicit conv)
// use for this shape when one is passed; 0 when the shape is not split
size_t linear_f32_split_floats(int M, int N, int K);
// taps: x rows may overlap (ldx < K) as launch_quantize_rows' taps view
void launch_linear_f32(float* out, int ldo, const float* x, int ldx, const float* W, int ldw,
                       const float* bias, int M, int N, int K, int act, int accumulate, float alpha,
                       hipStream_t st, float* work = nullptr, size_t work_floats = 0, bool taps = false);

// runtime.cpp
hipStream_t library_stream();  // stream of the host-pointer forms
bool device_is_gfx950();

}  // namespace hip
}  // namespace vla
