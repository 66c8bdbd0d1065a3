// graph.h - building blocks of the device-resident policy graphs: model-owned
// device memory, a linear layer that is int8 or fp32 as the model's int8 mask
// decides, the shared activation-quantization scratch, and HIP-graph replay of
// a whole forward pass.
//
// These replace the pieces of the reference's src/nn layer that the ACT, Octo
// and SmolVLA graphs drive: nn::Linear (src/nn/linear.h:40-99) with its int8
// state held in HBM, the shared quantization of MhaQKV (src/nn/attention.cpp:40-59)
// and nn::Scratch (src/nn/attention.h:17-22) as device buffers sized once.
#pragma once

#include "common.h"
#include "linear.h"

#include <cstdint>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace vla {
namespace hip {

// Device memory a model owns: every buffer is allocated at load (or on the
// first call with a new shape) and freed with the model.
class DeviceArena {
public:
    DeviceArena() = default;
    DeviceArena(const DeviceArena&) = delete;
    DeviceArena& operator=(const DeviceArena&) = delete;
    ~DeviceArena();
    void* raw(size_t bytes);  // zero-filled, 256-byte aligned
    template <class T>
    T* alloc(size_t n) {
        return static_cast<T*>(raw(n * sizeof(T)));
    }
    template <class T>
    T* upload(const T* host, size_t n) {
        T* d = alloc<T>(n);
        if (n) VLA_HIP_CHECK(hipMemcpy(d, host, n * sizeof(T), hipMemcpyHostToDevice));
        return d;
    }
    size_t bytes() const { return bytes_; }

private:
    std::vector<void*> blocks_;
    size_t bytes_ = 0;
};

// One block of rows of a (possibly row-concatenated) weight matrix, host fp32.
struct RowBlock {
    const float* W;     // [N, K]
    const float* bias;  // [N] or null (a null bias adds +0.0f, as the reference's epilogue does)
    int N;
};

// A linear layer as a model holds it. int8: device rows + per-row scales from
// the pack_weights_i8 quantizer (bit-identical per row whether or not rows are
// concatenated). fp32: the raw [N, K] weights. Row-concatenating layers that
// read the same input (q|k|v, k|v, gate|up) keeps one quantization of that
// input and one GEMM launch; each output block is bit-identical to its own
// layer's forward.
struct DLinear {
    int N = 0, K = 0;
    std::unique_ptr<vla_linear_i8> q8;
    float* W = nullptr;  // fp32 form [N, K]
    float* b = nullptr;  // fp32 form bias [N] (zeros where a block had none)
    bool int8() const { return q8 != nullptr; }
    int ldq() const { return q8 ? q8->ldw() : 0; }
    void init(DeviceArena& A, const std::vector<RowBlock>& blocks, int K, bool to_int8);
    void init(DeviceArena& A, const float* W, const float* bias, int N, int K, bool to_int8) {
        init(A, {{W, bias, N}}, K, to_int8);
    }
};

// Quantized activations: int8 rows [seq, ld] + per-row scales [seq].
struct QAct {
    int8_t* q = nullptr;
    float* s = nullptr;
    int ld = 0;
    bool panel = false;  // q in the panel layout (common.h) rather than [rows, ld]
};

// Per-model stream state: two activation-quantization slots shared by every
// int8 layer (the reference's thread_local xq/ascale, src/nn/linear.cpp:123-127),
// each [rows, ld_max] int8 + [rows] scales.
struct Ctx {
    hipStream_t st = nullptr;
    int8_t* xq[2] = {nullptr, nullptr};
    float* xs[2] = {nullptr, nullptr};
    size_t xq_bytes = 0;
    int xs_rows = 0;
    int32_t* split_ws = nullptr;  // split-K partial sums of the int8 GEMMs (8 MiB)
    size_t split_bytes = 0;
    // slot i laid out for a layer of row stride ld, for `rows` rows: the
    // panel layout when the rows feed the skinny GEMM (rows <= 128), else
    // row-major [rows, ld]
    QAct slot(int i, int ld, int rows) const;
    void alloc(class DeviceArena& A, int rows, int ld_max);
};

// The input of a linear layer: fp32 rows, or rows already quantized for it
// (q.ld == the layer's ldq()), or a row op not yet run (deferred: r, whose
// q / qs name the slot it quantizes into when it runs on its own).
struct In {
    const float* f = nullptr;
    int ldf = 0;
    bool taps = false;    // f's rows overlap (ldf < K): a 1-D convolution's taps view
    QAct q;               // valid when quantized or deferred
    bool quantized = false;
    bool deferred = false;
    RowQArgs r;
};

// x [seq, K] (row stride ldx) -> dst
void quantize(const Ctx& c, const QAct& dst, const float* x, int ldx, int seq, int K, bool taps = false);

// out[:, n0:n1] (+)= act(x W[n0:n1]^T + b). An int8 layer takes in.q when
// in.quantized, else quantizes in.f into slot 0; a deferred row op, or the
// quantization of fp32 rows, runs inside the GEMM (gemm_i8_rowop) for at most
// 16 rows when the shape allows it
// (K <= 2048, out apart from the rows read; VLA_HIP_ROWOP_FUSE=0 turns this
// off), else on its own first: the values are the same either way. acc != 0 adds into out (fmaf(alpha, v, out)
// for fp32 layers; the int8 epilogue adds v, alpha must be 1). With rope, the
// rotated columns come out rotated: inside the skinny GEMM's epilogue for an
// int8 layer of <= 128 rows without activation or accumulation (same floats
// as the separate rotation; VLA_HIP_ROPE_FUSE=0 or the int8-step probe turn it
// off), else by launch_rope_table after the layer.
// A RoPE rotation of the output's first `cols` columns (heads of hd columns)
// with the per-row (cos, sin) table cs [seq][hd / 2][2], as launch_rope_table
// applies it in place.
struct RopeEpi {
    const double* cs = nullptr;
    int cols = 0, hd = 0;
};

void linear(const Ctx& c, const DLinear& L, const In& in, float* out, int ldo, int seq, int act = 0,
            int acc = 0, int n0 = 0, int n1 = -1, float alpha = 1.0f, const RopeEpi* rope = nullptr);
inline void linear(const Ctx& c, const DLinear& L, float* out, int ldo, const float* x, int ldx,
                   int seq, int act = 0, int acc = 0, int n0 = 0, int n1 = -1, float alpha = 1.0f) {
    In in;
    in.f = x;
    in.ldf = ldx;
    linear(c, L, in, out, ldo, seq, act, acc, n0, n1, alpha);
}

// linear(c, L1, in1, out1, ldo1, seq) and linear(c, L2, in2, out2, ldo2, seq):
// two independent layers over the same rows (no activation, no accumulation),
// as one GEMM launch when both are int8 with quantized inputs and both take
// the unsplit skinny kernel (launch_gemm_i8_pair), else one after the other.
// The values are the same either way.
void linear_pair(const Ctx& c, const DLinear& L1, const In& in1, float* out1, int ldo1, const DLinear& L2,
                 const In& in2, float* out2, int ldo2, int seq);

// A row op (RowQArgs op / x / u / w / b / eps / rows / H) whose result feeds
// layer L: an int8 L gets it quantized in the same kernel, into `slot` (and
// fp32 rows into f when f is non-null); an fp32 L gets fp32 rows in f. For an
// int8 L without f, the op may be deferred to the linear() call that takes
// the returned In (the rows it reads must not change in between).
In rowop_for(const Ctx& c, const DLinear& L, RowQArgs r, float* f, int ldf, int slot);

// launch_rowq for the graphs: the same launch, plus the probe's bookkeeping
// when the probe is on.
void rowq(const RowQArgs& r, hipStream_t st);

// The int8-step probe (test support, vla_probe_*): while it is on, graphs run
// eagerly, no row op is fused into a GEMM (the values are the same either
// way), and each int8 GEMM of a pass is recorded on the host, up to
// max_records of them: the fp32 rows its activations were quantized from,
// the int8 activations and scales it read, its weight rows, scales and bias,
// and its output before and after the launch. Every record costs a device
// synchronization; nothing of this runs while the probe is off.
struct ProbeRecord {
    int M = 0, K = 0, N = 0, act = 0, acc = 0, has_bias = 0, has_src = 0;
    std::vector<float> src, as, before, after, ws, bias;  // src [M, K], before / after [M, N]
    std::vector<int8_t> xq, W;                            // xq [M, K], W [N, K]
};
void probe_begin(int max_records);
void probe_end();
bool probe_on();
const std::vector<ProbeRecord>& probe_records();

// Which keys a query may see (AttnArgs' mask fields): kind 0 none, 1 dense
// additive [sq, ldm], 2 causal (key j blocked when j > i + causal_offset),
// 3 group table (key j blocked when !allow[qg[i] * n_groups + kg[j]]).
struct MaskSpec {
    int kind = 0;
    const float* dense = nullptr;
    int ldm = 0;
    int causal_offset = 0;
    int n_groups = 0;
    const uint8_t* qg = nullptr;
    const uint8_t* kg = nullptr;
    const uint8_t* allow = nullptr;
};

// gqa attention over row-strided Q [sq, ldq], K/V [sk, ldk/ldv] -> out [sq, ldo]
void attend(hipStream_t st, float* out, int ldo, const float* Q, int ldq, const float* K, int ldk,
            const float* V, int ldv, int sq, int sk, int nq, int nkv, int hd, float scale,
            const MaskSpec& m);

// device copy of n floats (a kernel, so it records as a kernel node in a graph)
void copy_f32(float* dst, const float* src, int64_t n, hipStream_t st);
// dst rows [rows, cols] with strides from src rows
void copy_rows_f32(float* dst, int ldd, const float* src, int lds, int rows, int cols, hipStream_t st);

// Replays one forward pass as a HIP graph. The first call with a new key runs
// f eagerly (it also sets up lazily initialised kernels); the second captures
// f on the model's own stream; later calls launch the captured graph on the
// caller's stream. VLA_HIP_GRAPH=0 keeps every call eager.
class GraphReplay {
public:
    GraphReplay() = default;
    GraphReplay(const GraphReplay&) = delete;
    GraphReplay& operator=(const GraphReplay&) = delete;
    ~GraphReplay();
    void run(uint64_t key, hipStream_t own, hipStream_t caller, const std::function<void(hipStream_t)>& f);
    int nodes() const { return nodes_; }

private:
    void reset();
    uint64_t key_ = ~0ull;
    int calls_ = 0;
    int nodes_ = 0;
    hipGraph_t graph_ = nullptr;
    hipGraphExec_t exec_ = nullptr;
};

// rope_neox's per-token table (src/hal/common/norms.cpp:37-67): for token t,
// theta_0 = pos[t], theta_{i+1} = theta_i * base^(-2/head_dim) in double,
// entries (cos theta_i, sin theta_i) at [(t * head_dim/2 + i) * 2].
std::vector<double> rope_cos_sin(const int32_t* pos, int seq, int head_dim, float base);

// Host fp32 -> the bf16 the reference's converters store (top 16 bits), and back.
inline float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

}  // namespace hip
}  // namespace vla
