// graph.cpp - see graph.h.
#include "graph.h"

#include <cmath>
#include <cstdlib>
#include <fstream>
#include <map>
#include <sstream>

namespace vla {
namespace hip {

DeviceArena::~DeviceArena() {
    for (void* p : blocks_) (void)hipFree(p);
}

void* DeviceArena::raw(size_t bytes) {
    const size_t b = (bytes + 255) & ~(size_t)255;
    void* p = nullptr;
    VLA_HIP_CHECK(hipMalloc(&p, b ? b : 256));
    blocks_.push_back(p);
    VLA_HIP_CHECK(hipMemset(p, 0, b ? b : 256));
    // the fill runs on the null stream, which does not order with the
    // non-blocking streams the models launch on: wait for it, so no later
    // write into the block can land before the zeros
    VLA_HIP_CHECK(hipStreamSynchronize(nullptr));
    bytes_ += b;
    return p;
}

// ------------------------------------------------------------------ probe --

namespace {

struct ProbeSrc {
    std::vector<float> rows;  // [M, K], copied when the slot was written
    int M = 0, K = 0;
    int ldq = 0;              // the slot's int8 row stride (0: panel layout)
};

struct ProbeState {
    bool on = false;
    int max_records = 0;
    std::map<const void*, ProbeSrc> src;  // quantization slot -> the rows last quantized into it
    std::vector<ProbeRecord> recs;
    std::vector<void*> bufs;              // fp32 rows a row op wrote only for the probe
};

ProbeState& probe_state() {
    static ProbeState p;
    return p;
}

std::vector<float> d2h_f32(const float* src, int ld, int rows, int cols) {
    std::vector<float> h((size_t)rows * cols);
    if (rows > 0 && cols > 0 && ld >= cols)
        VLA_HIP_CHECK(hipMemcpy2D(h.data(), (size_t)cols * 4, src, (size_t)ld * 4, (size_t)cols * 4, rows,
                                  hipMemcpyDeviceToHost));
    else  // overlapping rows (a convolution's taps view): row by row
        for (int r = 0; r < rows && cols > 0; r++)
            VLA_HIP_CHECK(hipMemcpy(h.data() + (size_t)r * cols, src + (size_t)r * ld, (size_t)cols * 4,
                                    hipMemcpyDeviceToHost));
    return h;
}

// the int8 activations of a slot as [M, K] rows, from either layout
std::vector<int8_t> d2h_q(const QAct& q, int M, int K) {
    std::vector<int8_t> h((size_t)M * K);
    if (q.panel) {
        const int mp = panel_rows(M);
        std::vector<int8_t> raw(panel_bytes(M, K));
        VLA_HIP_CHECK(hipMemcpy(raw.data(), q.q, raw.size(), hipMemcpyDeviceToHost));
        for (int m = 0; m < M; m++)
            for (int k = 0; k < K; k++) h[(size_t)m * K + k] = raw[(size_t)(k / 64) * mp * 64 + m * 64 + k % 64];
    } else {
        VLA_HIP_CHECK(hipMemcpy2D(h.data(), K, q.q, q.ld, K, M, hipMemcpyDeviceToHost));
    }
    return h;
}

void probe_note(const void* slot, int ldq, const float* rows, int ld, int M, int K, hipStream_t st) {
    VLA_HIP_CHECK(hipStreamSynchronize(st));
    ProbeSrc s;
    s.rows = d2h_f32(rows, ld, M, K);
    s.M = M;
    s.K = K;
    s.ldq = ldq;
    probe_state().src[slot] = std::move(s);
}

// The fp32 rows behind int8 rows [q, q + M rows): the whole of a recorded
// slot, or (row-major slots) a run of its rows.
bool probe_source(const QAct& q, int M, int K, std::vector<float>& rows) {
    for (const auto& e : probe_state().src) {
        const ProbeSrc& s = e.second;
        const int8_t* base = static_cast<const int8_t*>(e.first);
        if (s.K != K) continue;
        if (q.q == base && s.M == M && (s.ldq == 0) == q.panel) {
            rows = s.rows;
            return true;
        }
        if (s.ldq == 0 || q.panel || q.ld != s.ldq || q.q < base) continue;
        const size_t off = (size_t)(q.q - base);
        if (off % s.ldq || off / s.ldq + M > (size_t)s.M) continue;
        const size_t r0 = off / s.ldq;
        rows.assign(s.rows.begin() + r0 * K, s.rows.begin() + (r0 + M) * K);
        return true;
    }
    return false;
}

}  // namespace

void probe_begin(int max_records) {
    probe_end();
    ProbeState& P = probe_state();
    P.on = true;
    P.max_records = max_records;
}

void probe_end() {
    ProbeState& P = probe_state();
    for (void* p : P.bufs) (void)hipFree(p);
    P.bufs.clear();
    P.src.clear();
    P.recs.clear();
    P.on = false;
}

bool probe_on() { return probe_state().on; }

const std::vector<ProbeRecord>& probe_records() { return probe_state().recs; }

void rowq(const RowQArgs& r0, hipStream_t st) {
    ProbeState& P = probe_state();
    if (!P.on) {
        launch_rowq(r0, st);
        return;
    }
    // the fp32 rows behind each quantization, written to probe buffers where
    // the graph itself keeps only the int8 form
    RowQArgs r = r0;
    auto rows_buf = [&]() {
        void* p = nullptr;
        VLA_HIP_CHECK(hipMalloc(&p, (size_t)r.rows * r.H * 4 + 16));
        P.bufs.push_back(p);
        return static_cast<float*>(p);
    };
    if (r.q && !r.out) {
        r.out = rows_buf();
        r.ldo = r.H;
    }
    if (r.q2 && r.add && !r.out2) {
        r.out2 = rows_buf();
        r.ldo2 = r.H;
    }
    launch_rowq(r, st);
    if (r.q) probe_note(r.q, r.q_panel ? 0 : r.ldq, r.out, r.ldo, r.rows, r.H, st);
    if (r.q2 && r.add) probe_note(r.q2, r.q_panel ? 0 : r.ldq2, r.out2, r.ldo2, r.rows, r.H, st);
}

void DLinear::init(DeviceArena& A, const std::vector<RowBlock>& blocks, int K_, bool to_int8) {
    VLA_REQUIRE(K_ > 0 && !blocks.empty(), "linear: need K > 0 and at least one block");
    int n = 0;
    for (const RowBlock& r : blocks) {
        VLA_REQUIRE(r.W && r.N > 0, "linear: null weights or empty block");
        n += r.N;
    }
    N = n;
    K = K_;
    std::vector<float> W32((size_t)N * K), b32((size_t)N, 0.0f);
    bool any_bias = false;
    size_t row = 0;
    for (const RowBlock& r : blocks) {
        std::memcpy(W32.data() + row * K, r.W, (size_t)r.N * K * sizeof(float));
        if (r.bias) {
            std::memcpy(b32.data() + row, r.bias, (size_t)r.N * sizeof(float));
            any_bias = true;
        }
        row += r.N;
    }
    if (to_int8) {
        q8 = vla_linear_i8::from_f32(W32.data(), any_bias ? b32.data() : nullptr, N, K);
    } else {
        W = A.upload(W32.data(), W32.size());
        b = any_bias ? A.upload(b32.data(), b32.size()) : nullptr;
    }
}

QAct Ctx::slot(int i, int ld, int rows) const {
    QAct a;
    a.q = xq[i];
    a.s = xs[i];
    a.ld = ld;
    a.panel = rows <= kPanelMaxRows;
    const size_t need = a.panel ? (size_t)panel_rows(rows) * ld : (size_t)rows * ld;
    VLA_REQUIRE(need <= xq_bytes && rows <= xs_rows, "graph: activation quantization scratch too small");
    return a;
}

void Ctx::alloc(DeviceArena& A, int rows, int ld_max) {
    // room for the panel layout's rows rounded up to 16 as well
    xq_bytes = (size_t)panel_rows(rows) * ld_max;
    xs_rows = rows;
    for (int i = 0; i < 2; i++) {
        xq[i] = A.alloc<int8_t>(xq_bytes);
        xs[i] = A.alloc<float>(rows);
    }
    split_bytes = (size_t)8 << 20;  // the most any split-K plan asks for
    split_ws = A.alloc<int32_t>(split_bytes / 4);
}

void quantize(const Ctx& c, const QAct& dst, const float* x, int ldx, int seq, int K, bool taps) {
    const size_t need = dst.panel ? (size_t)panel_rows(seq) * dst.ld : (size_t)seq * dst.ld;
    VLA_REQUIRE(need <= c.xq_bytes && seq <= c.xs_rows, "graph: activation quantization scratch too small");
    if (dst.panel) launch_quantize_rows_panel(x, ldx, dst.q, dst.s, seq, K, c.st, taps);
    else launch_quantize_rows(x, ldx, dst.q, dst.ld, dst.s, seq, K, c.st, taps);
    if (probe_on()) probe_note(dst.q, dst.panel ? 0 : dst.ld, x, ldx, seq, K, c.st);
}

static GemmArgs gemm_args(const DLinear& L, float* out, int ldo, int seq, int act, int acc, int n0, int n1) {
    const vla_linear_i8& q = *L.q8;
    GemmArgs a{};
    a.B = q.Wq() + (size_t)n0 * q.ldw();
    a.ldb = q.ldw();
    a.wscale = q.wscale() + n0;
    a.bias = q.bias() ? q.bias() + n0 : nullptr;
    a.out = out;
    a.ldo = ldo;
    a.M = seq;
    a.N = n1 - n0;
    a.K = L.K;
    a.act = act;
    a.accumulate = acc;
    return a;
}

// Whether linear() runs a row op inside the GEMM. Every block of the fused
// kernel applies the row op to all rows of its row group (all rows when the
// output is wide) (about 1000 VALU cycles per 720-wide
// RMSNorm row and SIMD, 3x that for a 2048-wide silu_gate row), so the fused
// kernel beats row kernel + GEMM only while each SIMD has a row or so: on
// MI355X at 16 rows it saved 4 us of 9.7 (RMSNorm, N = 4096, K = 720); at 50
// rows it lost 3 us (RMSNorm, N = 4096) to 22 us (silu_gate, K = 2048).
// The identity op (quantize only) was once worth repeating up to 64 rows
// (50 x 720 x 960: 8.6 us fused against 9.7 us as quantize + GEMM); since the
// panel quantizer keeps its row in registers, the separate pair wins there
// too (SmolVLA 8.54 -> 8.18 ms per chunk, same box), so every op fuses only up
// to 16 rows - or, for the identity op, wherever the fused kernel's row groups
// hold at most 16 rows (the 50-row o-projections, N = 720, 4 groups: 7.22 ->
// 7.03 ms per chunk, four alternating runs on one box). Fusing silu_gate
// (K = 2048) that way as well was slower: 7.33 -> 8.00 ms.
// VLA_HIP_ROWOP_FUSE=0 turns it off.
constexpr int kRowopFuseMaxRows = 16;

static bool fuse_rowop(int op, int seq, int K, int N) {
    static const bool on = [] {
        const char* e = std::getenv("VLA_HIP_ROWOP_FUSE");
        return !(e && e[0] == '0');
    }();
    const bool rows_ok =
        seq <= kRowopFuseMaxRows || (op == 0 && rowop_gemm_block_rows(seq, N) <= kRowopFuseMaxRows);
    return on && !probe_on() && rows_ok && rowop_gemm_fits(op, seq, K);
}

static bool overlaps(const float* p, size_t pn, const float* q, size_t qn) {
    return p < q + qn && q < p + pn;
}

// Runs the row op r inside the GEMM when the fused kernel takes this shape.
static bool try_rowop_gemm(const Ctx& c, const DLinear& L, const RowQArgs& r, float* out, int ldo, int seq,
                           int act, int acc, int n0, int n1) {
    if (!fuse_rowop(r.op, seq, L.K, n1 - n0) || L.q8->ldw() % 16) return false;
    const size_t on = (size_t)(seq - 1) * ldo + (n1 - n0);
    if (overlaps(out, on, r.x, (size_t)(seq - 1) * r.ldx + L.K)) return false;
    if (r.op == 3 && overlaps(out, on, r.u, (size_t)(seq - 1) * r.ldu + L.K)) return false;
    RowQArgs f = r;
    f.q = nullptr;
    f.qs = nullptr;
    f.q_panel = 0;
    launch_gemm_i8_rowop(f, gemm_args(L, out, ldo, seq, act, acc, n0, n1), c.st);
    return true;
}

static GemmArgs gemm_q_args(const Ctx& c, const DLinear& L, const QAct& x, float* out, int ldo, int seq, int act,
                            int acc, int n0, int n1) {
    const vla_linear_i8& q = *L.q8;
    VLA_REQUIRE(x.ld == q.ldw(), "linear: quantized input laid out for another layer width");
    GemmArgs a{};
    a.A = x.q;
    a.lda = x.ld;
    a.B = q.Wq() + (size_t)n0 * q.ldw();
    a.ldb = q.ldw();
    a.ascale = x.s;
    a.wscale = q.wscale() + n0;
    a.bias = q.bias() ? q.bias() + n0 : nullptr;
    a.out = out;
    a.ldo = ldo;
    a.M = seq;
    a.N = n1 - n0;
    a.K = L.K;
    a.act = act;
    a.accumulate = acc;
    a.a_panel = x.panel ? 1 : 0;
    a.split_ws = c.split_ws;
    a.split_bytes = c.split_bytes;
    return a;
}

static void gemm_q(const Ctx& c, const DLinear& L, const QAct& x, float* out, int ldo, int seq, int act,
                   int acc, int n0, int n1, const RopeEpi* rope = nullptr) {
    const vla_linear_i8& q = *L.q8;
    VLA_REQUIRE(x.ld == q.ldw(), "linear: quantized input laid out for another layer width");
    GemmArgs a{};
    a.A = x.q;
    a.lda = x.ld;
    a.B = q.Wq() + (size_t)n0 * q.ldw();
    a.ldb = q.ldw();
    a.ascale = x.s;
    a.wscale = q.wscale() + n0;
    a.bias = q.bias() ? q.bias() + n0 : nullptr;
    a.out = out;
    a.ldo = ldo;
    a.M = seq;
    a.N = n1 - n0;
    a.K = L.K;
    a.act = act;
    a.accumulate = acc;
    a.a_panel = x.panel ? 1 : 0;
    a.split_ws = c.split_ws;
    a.split_bytes = c.split_bytes;
    if (rope) {
        a.rope_cs = rope->cs;
        a.rope_cols = rope->cols;
        a.rope_hd = rope->hd;
    }
    ProbeState& P = probe_state();
    if (rope || !P.on || (int)P.recs.size() >= P.max_records) {
        launch_gemm_i8(a, c.st);
        return;
    }
    VLA_HIP_CHECK(hipStreamSynchronize(c.st));
    ProbeRecord rec;
    rec.M = seq;
    rec.K = L.K;
    rec.N = n1 - n0;
    rec.act = act;
    rec.acc = acc;
    rec.has_bias = q.bias() ? 1 : 0;
    rec.has_src = probe_source(x, seq, L.K, rec.src) ? 1 : 0;
    rec.xq = d2h_q(x, seq, L.K);
    rec.as = d2h_f32(x.s, seq, 1, seq);
    rec.W.resize((size_t)rec.N * L.K);
    VLA_HIP_CHECK(hipMemcpy2D(rec.W.data(), L.K, a.B, a.ldb, L.K, rec.N, hipMemcpyDeviceToHost));
    rec.ws = d2h_f32(a.wscale, rec.N, 1, rec.N);
    if (a.bias) rec.bias = d2h_f32(a.bias, rec.N, 1, rec.N);
    rec.before = d2h_f32(out, ldo, seq, rec.N);
    launch_gemm_i8(a, c.st);
    VLA_HIP_CHECK(hipStreamSynchronize(c.st));
    rec.after = d2h_f32(out, ldo, seq, rec.N);
    P.recs.push_back(std::move(rec));
}

// read at every call (graphs are recorded once per shape), so a test can build
// one model each way in the same process
static bool rope_fuse_on() {
    const char* e = std::getenv("VLA_HIP_ROPE_FUSE");
    return !(e && e[0] == '0');
}

void linear(const Ctx& c, const DLinear& L, const In& in, float* out, int ldo, int seq, int act, int acc,
            int n0, int n1, float alpha, const RopeEpi* rope) {
    if (n1 < 0) n1 = L.N;
    VLA_REQUIRE(0 <= n0 && n0 < n1 && n1 <= L.N, "linear: bad output row range");
    if (seq == 0) return;
    if (rope) {
        VLA_REQUIRE(rope->cs && rope->hd > 0 && rope->hd % 2 == 0 && rope->cols > 0 && rope->cols % rope->hd == 0 &&
                        rope->cols <= n1 - n0,
                    "linear: rotation of whole heads within the output columns");
        const bool fused = rope_fuse_on() && !probe_on() && L.int8() && seq <= kPanelMaxRows && act == 0 &&
                           acc == 0 && rope->hd % 16 == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0 &&
                           L.q8->ldw() % 16 == 0;
        if (!fused) {
            linear(c, L, in, out, ldo, seq, act, acc, n0, n1, alpha);
            launch_rope_table(out, ldo, rope->cs, seq, rope->cols / rope->hd, rope->hd, c.st);
            return;
        }
        if (in.deferred) {
            VLA_REQUIRE(in.r.rows == seq && in.r.H == L.K && in.q.ld == L.ldq(),
                        "linear: deferred row op made for another layer or row count");
            rowq(in.r, c.st);
            gemm_q(c, L, in.q, out, ldo, seq, 0, 0, n0, n1, rope);
        } else if (in.quantized) {
            gemm_q(c, L, in.q, out, ldo, seq, 0, 0, n0, n1, rope);
        } else {
            VLA_REQUIRE(in.f, "linear: no input");
            const QAct s0 = c.slot(0, L.ldq(), seq);
            quantize(c, s0, in.f, in.ldf, seq, L.K);
            gemm_q(c, L, s0, out, ldo, seq, 0, 0, n0, n1, rope);
        }
        return;
    }
    if (L.int8() && act == 4) {
        // the int8 epilogue has no silu: the GEMM, then silu over the block in
        // place (the reference's Linear::forward then silu(), diffusion.cpp:24-26)
        VLA_REQUIRE(acc == 0, "linear: int8 silu layers cannot accumulate");
        linear(c, L, in, out, ldo, seq, 0, 0, n0, n1, alpha);
        const int w = n1 - n0;
        if (ldo == w || seq == 1) {
            launch_act(out, (int64_t)seq * w, 4, c.st);
        } else {
            for (int r = 0; r < seq; r++) launch_act(out + (size_t)r * ldo, w, 4, c.st);
        }
        return;
    }
    if (L.int8()) {
        VLA_REQUIRE(alpha == 1.0f, "linear: the int8 epilogue accumulates with alpha = 1 only");
        VLA_REQUIRE(act <= 3, "linear: the int8 epilogue has no silu");
        if (in.deferred) {
            VLA_REQUIRE(in.r.rows == seq && in.r.H == L.K && in.q.ld == L.ldq(),
                        "linear: deferred row op made for another layer or row count");
            if (try_rowop_gemm(c, L, in.r, out, ldo, seq, act, acc, n0, n1)) return;
            rowq(in.r, c.st);
            gemm_q(c, L, in.q, out, ldo, seq, act, acc, n0, n1);
        } else if (in.quantized) {
            gemm_q(c, L, in.q, out, ldo, seq, act, acc, n0, n1);
        } else {
            VLA_REQUIRE(in.f, "linear: no input");
            if (seq <= 64 && in.ldf % 4 == 0 && (reinterpret_cast<uintptr_t>(in.f) & 15) == 0) {
                RowQArgs r;  // identity row op: quantize_rows_panel's bytes and scales
                r.op = 0;
                r.x = in.f;
                r.ldx = in.ldf;
                r.rows = seq;
                r.H = L.K;
                r.taps = in.taps ? 1 : 0;
                if (try_rowop_gemm(c, L, r, out, ldo, seq, act, acc, n0, n1)) return;
            }
            const QAct s0 = c.slot(0, L.ldq(), seq);
            quantize(c, s0, in.f, in.ldf, seq, L.K, in.taps);
            gemm_q(c, L, s0, out, ldo, seq, act, acc, n0, n1);
        }
    } else {
        VLA_REQUIRE(in.f, "linear: an fp32 layer needs fp32 input rows");
        launch_linear_f32(out, ldo, in.f, in.ldf, L.W + (size_t)n0 * L.K, L.K, L.b ? L.b + n0 : nullptr, seq,
                          n1 - n0, L.K, act, acc, alpha, c.st, nullptr, 0, in.taps);
    }
}

void linear_pair(const Ctx& c, const DLinear& L1, const In& in1, float* out1, int ldo1, const DLinear& L2,
                 const In& in2, float* out2, int ldo2, int seq) {
    if (seq > 0 && !probe_on() && L1.int8() && L2.int8() && in1.quantized && in2.quantized &&
        in1.q.ld == L1.ldq() && in2.q.ld == L2.ldq()) {
        const GemmArgs a1 = gemm_q_args(c, L1, in1.q, out1, ldo1, seq, 0, 0, 0, L1.N);
        const GemmArgs a2 = gemm_q_args(c, L2, in2.q, out2, ldo2, seq, 0, 0, 0, L2.N);
        if (launch_gemm_i8_pair(a1, a2, c.st)) return;
    }
    linear(c, L1, in1, out1, ldo1, seq);
    linear(c, L2, in2, out2, ldo2, seq);
}

In rowop_for(const Ctx& c, const DLinear& L, RowQArgs r, float* f, int ldf, int slot) {
    In in;
    r.out = f;
    r.ldo = ldf;
    if (L.int8()) {
        in.q = c.slot(slot, L.ldq(), r.rows);
        in.quantized = true;
        r.q = in.q.q;
        r.ldq = in.q.ld;
        r.qs = in.q.s;
        r.q_panel = in.q.panel ? 1 : 0;
    } else {
        VLA_REQUIRE(f, "graph: an fp32 consumer needs the fp32 rows");
    }
    in.f = f;
    in.ldf = ldf;
    if (L.int8() && !f && !r.add && fuse_rowop(r.op, r.rows, L.K, L.N)) {
        in.quantized = false;
        in.deferred = true;
        in.r = r;
        return in;
    }
    rowq(r, c.st);
    return in;
}

void attend(hipStream_t st, float* out, int ldo, const float* Q, int ldq, const float* K, int ldk,
            const float* V, int ldv, int sq, int sk, int nq, int nkv, int hd, float scale,
            const MaskSpec& m) {
    AttnArgs a{};
    a.out = out;
    a.ldo = ldo;
    a.Q = Q;
    a.ldq = ldq;
    a.K = K;
    a.ldk = ldk;
    a.V = V;
    a.ldv = ldv;
    a.seq_q = sq;
    a.seq_k = sk;
    a.n_q = nq;
    a.n_kv = nkv;
    a.head_dim = hd;
    a.scale = scale;
    a.mask_kind = m.kind;
    a.mask = m.dense;
    a.ldm = m.ldm;
    a.causal_offset = m.causal_offset;
    a.n_groups = m.n_groups;
    a.q_group = m.qg;
    a.k_group = m.kg;
    a.allow = m.allow;
    launch_attention(a, st);
}

void copy_f32(float* dst, const float* src, int64_t n, hipStream_t st) {
    VLA_REQUIRE(n >= 0 && n < (int64_t)1 << 31, "copy: size out of range");
    launch_copy_rows(dst, (int)n, src, (int)n, 1, (int)n, st);
}

void copy_rows_f32(float* dst, int ldd, const float* src, int lds, int rows, int cols, hipStream_t st) {
    launch_copy_rows(dst, ldd, src, lds, rows, cols, st);
}

// ---------------------------------------------------------------- replay --

GraphReplay::~GraphReplay() { reset(); }

void GraphReplay::reset() {
    if (exec_) (void)hipGraphExecDestroy(exec_);
    if (graph_) (void)hipGraphDestroy(graph_);
    exec_ = nullptr;
    graph_ = nullptr;
    nodes_ = 0;
}

static bool graphs_enabled() {
    static const bool on = [] {
        const char* e = std::getenv("VLA_HIP_GRAPH");
        return !(e && e[0] == '0');
    }();
    return on;
}

void GraphReplay::run(uint64_t key, hipStream_t own, hipStream_t caller,
                      const std::function<void(hipStream_t)>& f) {
    if (key != key_) {
        reset();
        key_ = key;
        calls_ = 0;
    }
    calls_++;
    if (!graphs_enabled() || calls_ == 1 || probe_on()) {
        // eager: on the caller's stream, ordered with its other work
        f(caller);
        return;
    }
    if (!exec_) {
        // the caller's stream may be the null stream, which cannot be captured
        VLA_HIP_CHECK(hipStreamSynchronize(caller));
        VLA_HIP_CHECK(hipStreamBeginCapture(own, hipStreamCaptureModeThreadLocal));
        try {
            f(own);
        } catch (...) {
            hipGraph_t g = nullptr;
            (void)hipStreamEndCapture(own, &g);
            if (g) (void)hipGraphDestroy(g);
            throw;
        }
        VLA_HIP_CHECK(hipStreamEndCapture(own, &graph_));
        size_t n = 0;
        VLA_HIP_CHECK(hipGraphGetNodes(graph_, nullptr, &n));
        nodes_ = (int)n;
        VLA_HIP_CHECK(hipGraphInstantiate(&exec_, graph_, nullptr, nullptr, 0));
    }
    VLA_HIP_CHECK(hipGraphLaunch(exec_, caller));
}

std::vector<double> rope_cos_sin(const int32_t* pos, int seq, int head_dim, float base) {
    const int half = head_dim / 2;
    const double theta_scale = std::pow((double)base, -2.0 / head_dim);
    std::vector<double> cs((size_t)seq * half * 2);
    for (int t = 0; t < seq; t++) {
        double theta = (double)pos[t];
        for (int i = 0; i < half; i++) {
            cs[((size_t)t * half + i) * 2] = std::cos(theta);
            cs[((size_t)t * half + i) * 2 + 1] = std::sin(theta);
            theta *= theta_scale;
        }
    }
    return cs;
}

}  // namespace hip
}  // namespace vla
