// noalloc.hip - vla_dense_linear_i8_noalloc_dev: vla_dense_linear_i8_dev
// without caller scratch and without any allocation, for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).
//
// Its scratch (the quantized activations, their scales and the split-K int32
// partial sums) lives in one file-scope __device__ array of fixed size. Each
// GPU holds its own copy until the process ends. Host code never uses the
// array's name as an address: on the first call on a device, with that device
// current, hipGetSymbolAddress gives that device's address, kept per device
// and passed to the kernels like any other buffer.
//
// Every call on a device shares that device's array and leaves its contents
// behind; calls that overlap on one device (two streams, two threads) race.
// Nothing in it has to start at zero: the quantizer writes every byte the GEMM
// reads (the zero pad [K, ldq) of each row, the whole last 64-byte panel) and
// the split-K pass writes every partial sum before the reduce reads it.
#include "vla_simd_hip.h"

#include "common.h"
#include "runtime.h"

#include <mutex>

namespace vla {
namespace hip {
namespace {

// Layout of the array: [xq | ascale | split-K partial sums].
constexpr size_t kXqBytes = (size_t)32 << 20;      // seq x ldq int8 (8192 x 4096 fits)
constexpr int kMaxRows = 65536;                    // ascale floats
constexpr size_t kScaleBytes = (size_t)kMaxRows * 4;
constexpr size_t kSplitBytes = (size_t)8 << 20;    // the most any split-K plan asks for
constexpr size_t kScratchBytes = kXqBytes + kScaleBytes + kSplitBytes;

__device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
char* g_ptr[kMaxDevices] = {};

// This device's address of `scratch`, looked up once per device.
char* scratch_ptr() {
    int dev = -1;
    VLA_HIP_CHECK(hipGetDevice(&dev));
    VLA_REQUIRE(dev >= 0 && dev < kMaxDevices, "device index out of range");
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[dev]) {
        void* p = nullptr;
        VLA_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        VLA_REQUIRE(p != nullptr, "hipGetSymbolAddress returned no address for the scratch array");
        g_ptr[dev] = static_cast<char*>(p);
    }
    return g_ptr[dev];
}

}  // namespace
}  // namespace hip
}  // namespace vla

using namespace vla::hip;

extern "C" {

VLA_API int64_t vla_dense_linear_i8_noalloc_max_bytes(void) { return (int64_t)kXqBytes; }

VLA_API int32_t vla_dense_linear_i8_noalloc_dev(float* out, int32_t ldo, const float* x, int32_t ldx,
                                                const int8_t* Wq, int32_t ldw, const float* wscale,
                                                const float* bias, int32_t seq, int32_t N, int32_t K,
                                                int32_t act, int32_t accumulate, void* stream) {
    return guarded("vla_dense_linear_i8_noalloc_dev", [&] {
        VLA_REQUIRE(seq >= 0 && N > 0 && K > 0, "need seq >= 0, N > 0, K > 0");
        VLA_REQUIRE(K <= kMaxI8K, "K exceeds the int8 accumulator bound INT_MAX/(255*127)");
        VLA_REQUIRE(seq == 0 || (out && x && Wq && wscale), "null buffer");
        VLA_REQUIRE(seq <= kMaxRows, "seq exceeds the 65536 rows of the allocation-free scratch");
        if (seq == 0) return;
        // the panel layout for up to 128 rows when the GEMM can take it (what
        // the skinny GEMM reads fastest), else rows of i8_kpad(K) rounded to
        // 16 bytes; the values are the same either way
        const bool panel = seq <= kPanelMaxRows && ldw % 16 == 0 && aligned(Wq, 16) && aligned(out, 16);
        const int ldq = (kpad4(K) + 15) & ~15;
        const size_t xq_need = panel ? panel_bytes(seq, K) : (size_t)seq * ldq;
        VLA_REQUIRE(xq_need <= kXqBytes,
                    "seq x K exceeds the 32 MiB of quantized activations the allocation-free scratch holds");
        char* base = scratch_ptr();
        int8_t* xq = reinterpret_cast<int8_t*>(base);
        float* sa = reinterpret_cast<float*>(base + kXqBytes);
        int32_t* ws = reinterpret_cast<int32_t*>(base + kXqBytes + kScaleBytes);
        hipStream_t st = static_cast<hipStream_t>(stream);
        if (panel) launch_quantize_rows_panel(x, ldx, xq, sa, seq, K, st);
        else launch_quantize_rows(x, ldx, xq, ldq, sa, seq, K, st);
        GemmArgs a{};
        a.A = xq;
        a.lda = panel ? 0 : ldq;
        a.a_panel = panel ? 1 : 0;
        a.B = Wq;
        a.ldb = ldw;
        a.ascale = sa;
        a.wscale = wscale;
        a.bias = bias;
        a.out = out;
        a.ldo = ldo;
        a.M = seq;
        a.N = N;
        a.K = K;
        a.act = act;
        a.accumulate = accumulate;
        a.split_ws = ws;
        a.split_bytes = kSplitBytes;
        launch_gemm_i8(a, st);
    });
}

}  // extern "C"
