// ops_hip.cpp - the reference's op layer (namespace tcpu, src/ops/quant_ops.h,
// src/ops/lm_ops.h, src/ops/conv_ops.h) implemented over libvla_simd_hip.so.
//
// This is the file a maintainer adds to the reference as src/hal/hip/ops_hip.cpp
// to put its int8 linear + attention hot path on an MI355X: it is compiled
// against the reference's own headers and linked in place of the CPU
// translation units that define these functions (src/hal/common/gemm_i8.cpp,
// src/hal/avx2/gemm_i8.cpp, src/hal/avx2/attn.cpp, src/hal/common/attn.cpp,
// src/hal/common/norms.cpp, src/hal/common/eltwise.cpp). Everything else of the
// reference (nn::Linear, nn::MhaQKV, nn::EncoderLayer, the fp32 GEMMs, the
// model graphs) links against it unchanged. oracle/Makefile's ref_hip target
// builds exactly that set.
//
// Contract kept from the reference's op layer:
//   - pointers are caller-owned host memory and every call is synchronous (the
//     library's host-pointer forms upload, run and download); the int8 weights
//     of a packed layer stay resident on the device (below), so a layer's
//     forward moves only its activations and outputs;
//   - weights are packed once by pack_weights_i8 into a buffer of
//     packed_i8_words(N, K) int32 words: here the device row layout [N, Kp]
//     int8 (the i8 MFMA is signed x signed) followed by the int32 row-sum
//     table i8_rowsums returns, the same word count as the reference's panels;
//   - xq/ascale scratch of dense_linear_i8 receives the quantized rows, as the
//     reference's does;
//   - the reference asserts its preconditions; here a failed call throws
//     std::runtime_error with vla_last_error(), which the reference's C ABI
//     turns into VLA_ERR_EXCEPTION (include/vla_simd.h:15-20).
// Functions of lm_ops.h outside the hot path (mha_attention_bias, silu, mish,
// the fp32 and bf16 GEMMs) are not defined here: they stay the reference's
// CPU code.

#include "hal/common/layout.h"
#include "ops/conv_ops.h"
#include "ops/lm_ops.h"
#include "ops/quant_ops.h"

#include "vla_simd_hip.h"

#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace tcpu {

namespace {

void ok(int32_t status, const char* what) {
    if (status != VLA_OK) throw std::runtime_error(std::string(what) + ": " + vla_last_error());
}

// The key rows [seq_k, n_kv * head_dim] the device attention reads. nn::MhaQKV
// hands over only the transposed keys when its key projection writes them
// that way (Linear::kt_ok on an x86 build, attention.cpp:28-66): K_pre is
// [n_kv][head_dim][hal::kt_stride(seq_k)] (hal/common/layout.h:21-52), so the
// rows are gathered back from it.
const float* key_rows(std::vector<float>& tmp, const float* K, const float* K_pre, int seq_k, int n_kv,
                      int head_dim) {
    if (K || !K_pre) return K;
    const int ldk = hal::kt_stride(seq_k);
    tmp.resize((size_t)seq_k * n_kv * head_dim);
    for (int g = 0; g < n_kv; g++)
        for (int d = 0; d < head_dim; d++) {
            const float* col = K_pre + ((size_t)g * head_dim + d) * ldk;
            for (int j = 0; j < seq_k; j++) tmp[((size_t)j * n_kv + g) * head_dim + d] = col[j];
        }
    return tmp.data();
}

// ------------------------------------------------------ weight residency --
//
// nn::Linear and nn::Conv pack their int8 weights once, into a buffer each
// owns for its lifetime (pack_weights_i8 at linear.cpp:97-99 and
// conv.cpp:46), and pass the same Wq / wscale pointers on every forward
// (linear.cpp:121-133, 170-172; conv.cpp:59). The packing call here quantizes
// on the device and keeps that copy resident, keyed by the Wq address:
//   - a later pack into the same address replaces the entry (a layer
//     initialised again, or a freed buffer reused by a new layer);
//   - every forward first compares the buffer's row-sum table (written only
//     by pack_weights_i8, after the rows) and its wscale with the packed
//     values (8 N bytes); any difference, an unknown address or a different
//     N / K takes the upload-per-call path, which is always correct;
//   - the bias comes with each call: the entry keeps the address and values
//     of the one it holds and uploads a new one only when they differ;
//   - at most VLA_HIP_RESIDENT_MB (default 65536) MiB of int8 rows are made
//     resident; packs beyond it stay upload-per-call.
// Entries live until the process ends or their address is packed again (the
// op layer is not told when a layer is destroyed).
struct Resident {
    vla_linear_i8* lin = nullptr;
    int N = 0, K = 0;
    std::vector<int32_t> rowsums;
    std::vector<float> wscale;
    bool has_bias = false;
    const float* bias_ptr = nullptr;
    std::vector<float> bias;
};

struct ResidentTable {
    std::mutex mu;
    std::unordered_map<const int8_t*, Resident> map;
    size_t bytes = 0;
};

// never destroyed: its device memory goes with the process (freeing it from a
// static destructor could run after the HIP runtime has shut down)
ResidentTable& resident_table() {
    static ResidentTable* t = new ResidentTable();
    return *t;
}

size_t resident_limit() {
    const char* e = std::getenv("VLA_HIP_RESIDENT_MB");
    const long long mb = e && *e ? std::atoll(e) : 65536;
    return mb > 0 ? (size_t)mb << 20 : 0;
}

void drop_resident(ResidentTable& t, const int8_t* Wq) {
    auto it = t.map.find(Wq);
    if (it == t.map.end()) return;
    t.bytes -= (size_t)it->second.N * (size_t)vla_i8_kpad(it->second.K);
    vla_linear_i8_free(it->second.lin);
    t.map.erase(it);
}

// The resident layer of a packed buffer, with the call's bias in place, or
// null (not packed here, changed since, or another shape). Called with the
// table locked.
vla_linear_i8* find_resident(ResidentTable& t, const int8_t* Wq, const float* wscale, const float* bias, int N,
                             int K) {
    auto it = t.map.find(Wq);
    if (it == t.map.end()) return nullptr;
    Resident& r = it->second;
    const size_t Kp = (size_t)vla_i8_kpad(K);
    if (r.N != N || r.K != K || !wscale) return nullptr;
    if (std::memcmp(Wq + (size_t)N * Kp, r.rowsums.data(), (size_t)N * 4) != 0 ||
        std::memcmp(wscale, r.wscale.data(), (size_t)N * 4) != 0)
        return nullptr;
    const bool same_bias = bias ? (r.has_bias && r.bias_ptr == bias &&
                                   std::memcmp(bias, r.bias.data(), (size_t)N * 4) == 0)
                                : !r.has_bias;
    if (!same_bias) {
        ok(vla_linear_i8_set_bias(r.lin, bias), "pack_weights_i8 (bias)");
        r.has_bias = bias != nullptr;
        r.bias_ptr = bias;
        if (bias) r.bias.assign(bias, bias + N);
        else r.bias.clear();
    }
    return r.lin;
}

}  // namespace

// ---------------------------------------------------------- quant_ops.h --

bool int8_gemm_available() { return vla_int8_available() == 1; }  // quant_ops.h:41

int i8_kpad(int K) { return vla_i8_kpad(K); }  // quant_ops.h:45

// quant_ops.h:55: N rows of i8_kpad(K) bytes, then N int32 row sums
size_t packed_i8_words(int N, int K) { return (size_t)N * (size_t)i8_kpad(K) / 4 + (size_t)N; }

// quant_ops.h:56: the per-row absmax quantizer (on the device), rows [N, Kp]
// zero-padded, then the exact row sums the reference stores after its panels.
// The quantized rows stay resident on the device for this buffer's forwards.
void pack_weights_i8(const float* W, int8_t* Wq, float* wscale, int N, int K) {
    const int Kp = i8_kpad(K);
    ResidentTable& t = resident_table();
    std::lock_guard<std::mutex> lk(t.mu);
    drop_resident(t, Wq);
    const size_t rows = (size_t)N * Kp;
    vla_linear_i8* lin = nullptr;
    if (t.bytes + rows <= resident_limit()) {
        lin = vla_linear_i8_create(W, nullptr, N, K);
        if (!lin) ok(VLA_ERR_EXCEPTION, "pack_weights_i8");
        const int32_t st = vla_linear_i8_download(lin, Wq, Kp, wscale);
        if (st != VLA_OK) vla_linear_i8_free(lin);
        ok(st, "pack_weights_i8");
    } else {
        ok(vla_pack_weights_i8(W, Wq, wscale, N, K), "pack_weights_i8");
    }
    int32_t* sums = reinterpret_cast<int32_t*>(Wq + rows);
    for (int n = 0; n < N; n++) {
        int32_t s = 0;
        for (int k = 0; k < K; k++) s += Wq[(size_t)n * Kp + k];
        sums[n] = s;
    }
    if (lin) {
        Resident r;
        r.lin = lin;
        r.N = N;
        r.K = K;
        r.rowsums.assign(sums, sums + N);
        r.wscale.assign(wscale, wscale + N);
        t.map.emplace(Wq, std::move(r));
        t.bytes += rows;
    }
}

// quant_ops.h:63
const int32_t* i8_rowsums(const int8_t* Wq, int N, int K) {
    return reinterpret_cast<const int32_t*>(Wq + (size_t)N * i8_kpad(K));
}

// quant_ops.h:76
void quantize_act_i8(const float* x, int8_t* xq, float* ascale, int seq, int K) {
    ok(vla_quantize_act_i8(x, xq, ascale, seq, K), "quantize_act_i8");
}

// quant_ops.h:80
void quantize_span_i8(const float* x, int8_t* q, size_t n, float inv) {
    ok(vla_quantize_span_i8(x, q, (int64_t)n, inv), "quantize_span_i8");
}

// quant_ops.h:83
void dense_linear_i8_pre(float* out, const int8_t* xq, const float* ascale, const int8_t* Wq,
                         const float* wscale, const float* bias, int seq, int N, int K) {
    ResidentTable& t = resident_table();
    std::lock_guard<std::mutex> lk(t.mu);
    if (vla_linear_i8* lin = find_resident(t, Wq, wscale, bias, N, K)) {
        ok(vla_linear_i8_forward_quantized(lin, out, xq, i8_kpad(K), ascale, seq), "dense_linear_i8_pre");
        return;
    }
    ok(vla_dense_linear_i8_pre(out, xq, ascale, Wq, wscale, bias, seq, N, K), "dense_linear_i8_pre");
}

// quant_ops.h:69-72: the quantized rows land in the caller's scratch first
void dense_linear_i8(float* out, const float* x, const int8_t* Wq, const float* wscale, const float* bias,
                     int seq, int N, int K, int8_t* xq_scratch, float* ascale_scratch) {
    {
        ResidentTable& t = resident_table();
        std::lock_guard<std::mutex> lk(t.mu);
        if (vla_linear_i8* lin = find_resident(t, Wq, wscale, bias, N, K)) {
            ok(vla_linear_i8_forward(lin, out, x, seq, xq_scratch, i8_kpad(K), ascale_scratch), "dense_linear_i8");
            return;
        }
    }
    quantize_act_i8(x, xq_scratch, ascale_scratch, seq, K);
    dense_linear_i8_pre(out, xq_scratch, ascale_scratch, Wq, wscale, bias, seq, N, K);
}

// quant_ops.h:89-91: the scalar statement of the same call, on the host, over
// this backend's row layout: exact int32 dot, then fma(acc * ws, sa, bias)
// (gemm_i8.cpp:270-278). The device GEMM must equal it bit for bit.
void dense_linear_i8_ref(float* out, const int8_t* xq, const float* ascale, const int8_t* Wq,
                         const float* wscale, const float* bias, int seq, int N, int K) {
    const int Kp = i8_kpad(K);
    for (int t = 0; t < seq; t++)
        for (int n = 0; n < N; n++) {
            int32_t acc = 0;
            for (int k = 0; k < K; k++) acc += (int32_t)xq[(size_t)t * Kp + k] * (int32_t)Wq[(size_t)n * Kp + k];
            const float p = (float)acc * wscale[n];
            out[(size_t)t * N + n] = std::fma(p, ascale[t], bias ? bias[n] : 0.0f);
        }
}

// ------------------------------------------------------------- lm_ops.h --

void rmsnorm(float* out, const float* x, const float* w, int seq, int hidden, float eps) {  // lm_ops.h:21
    ok(vla_rmsnorm(out, x, w, seq, hidden, eps), "rmsnorm");
}

void rope_neox(float* x, const int* pos, int seq, int n_heads, int head_dim, float base) {  // lm_ops.h:26
    ok(vla_rope_neox(x, pos, seq, n_heads, head_dim, base), "rope_neox");
}

// lm_ops.h:33: K rows, or (K null) the transposed K_pre
void gqa_attention_masked(float* out, const float* Q, const float* K, const float* V, int seq_q, int seq_k,
                          int n_q, int n_kv, int head_dim, float scale, const float* mask, const float* K_pre) {
    std::vector<float> tmp;
    const float* Kr = key_rows(tmp, K, K_pre, seq_k, n_kv, head_dim);
    ok(vla_gqa_attention_masked(out, Q, Kr, V, seq_q, seq_k, n_q, n_kv, head_dim, scale, mask),
       "gqa_attention_masked");
}

void gqa_attention_dense(float* out, const float* Q, const float* K, const float* V, int seq_q, int seq_k,
                         int n_q, int n_kv, int head_dim, float scale, const float* K_pre) {  // lm_ops.h:43
    std::vector<float> tmp;
    const float* Kr = key_rows(tmp, K, K_pre, seq_k, n_kv, head_dim);
    ok(vla_gqa_attention_dense(out, Q, Kr, V, seq_q, seq_k, n_q, n_kv, head_dim, scale), "gqa_attention_dense");
}

void silu_gate(float* out, const float* g, const float* u, int n) {  // lm_ops.h:55
    ok(vla_silu_gate(out, g, u, n), "silu_gate");
}

void layernorm(float* out, const float* x, const float* w, const float* b, int seq, int hidden,
               float eps) {  // lm_ops.h:61
    ok(vla_layernorm(out, x, w, b, seq, hidden, eps), "layernorm");
}

void gelu_tanh(float* x, int n) { ok(vla_gelu_tanh(x, n), "gelu_tanh"); }  // lm_ops.h:64
void gelu_erf(float* x, int n) { ok(vla_gelu_erf(x, n), "gelu_erf"); }     // lm_ops.h:70
void relu(float* x, int n) { ok(vla_relu(x, n), "relu"); }                 // lm_ops.h:73

// ----------------------------------------------------------- conv_ops.h --

// conv_ops.h:31: Wq / wscale as pack_weights_i8 wrote them for [Cout, k*k*Cin];
// the device keeps its own im2col workspace, so xq_scratch is not touched
void conv2d_i8(float* out, const float* x, const int8_t* Wq, const float* wscale, const float* bias, int H,
               int Wd, int Cin, int Cout, int k, int stride, int pad, std::vector<int8_t>&) {
    {
        ResidentTable& t = resident_table();
        std::lock_guard<std::mutex> lk(t.mu);
        if (vla_linear_i8* lin = find_resident(t, Wq, wscale, bias, Cout, k * k * Cin)) {
            ok(vla_conv2d_i8_resident(lin, out, x, H, Wd, Cin, k, stride, pad), "conv2d_i8");
            return;
        }
    }
    ok(vla_conv2d_i8(out, x, Wq, wscale, bias, H, Wd, Cin, Cout, k, stride, pad), "conv2d_i8");
}

}  // namespace tcpu
