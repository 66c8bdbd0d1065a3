// gemm_i8.hip - W8A8 GEMM on the CDNA4 int8 matrix cores (gfx950).
//
// out[m,n] = fma((float)acc[m,n] * wscale[n], ascale[m], bias[n] or 0)
// acc[m,n] = sum_k xq[m,k] * Wq[n,k]   (exact int32)
//
// This is the contract of the reference's dense_linear_i8_pre
// (src/hal/common/gemm_i8.cpp:262-281, the epilogue expression at :278; the
// AVX-VNNI kernel src/hal/avx2/gemm_i8.cpp:88-105 computes the same value).
// Integer accumulation is exact and order-free, so any tiling, k-split or MFMA
// lane order gives the same int32; the fp32 epilogue is then one rounded
// product and one fma per output, in the reference's order. Contraction is off
// in this file so the product stays a separate rounding.
//
// Kernels
//   gemm_i8_tiled   BM x BN block tile, 4 waves in a WM x WN grid, K staged
//                   through LDS in BK-byte slabs, double buffered (global loads
//                   of slab k+1 are in flight while slab k feeds the MFMAs).
//                   v_mfma_i32_16x16x64_i8: lane l supplies 16 contiguous bytes
//                   of row (l % 16) at k offset 16*(l / 16) for both operands,
//                   so whatever k order the unit uses inside one instruction it
//                   pairs equal k on both sides. Output lane l holds column
//                   l % 16, rows 4*(l/16) + r.
//                   LDS rows are padded by 16 bytes so the 16 rows one
//                   ds_read_b128 touches fall on distinct bank groups.
//                   Workgroups are remapped so each XCD (the hardware deals
//                   workgroup i to XCD i % 8) owns a contiguous run of tiles,
//                   grouped 8 tile-rows deep, which keeps the A and B panels a
//                   run shares in that XCD's L2.
//   gemm_i8_skinny  M <= 128 (action chunks, decode rows): one block owns a
//                   16*FN-column slab of the output and every row; its waves
//                   split K, stream Wq straight from HBM into MFMA registers
//                   (each weight byte is read once) and sum their int32
//                   partials with LDS atomics before one epilogue. A second
//                   grid dimension splits K across blocks when the slab count
//                   alone cannot fill the chip; those partials meet in a global
//                   int32 workspace and the last block of a slab runs the
//                   epilogue.

#include "act.h"
#include "common.h"

#pragma clang fp contract(off)

namespace vla {
namespace hip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mfma_i8(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Bytes [K, ...) of a word that starts at byte kk are zeroed.
__device__ __forceinline__ int mask_word(int w, int kk, int K) {
    const int valid = K - kk;
    if (valid >= 4) return w;
    if (valid <= 0) return 0;
    return w & (int)((1u << (8 * valid)) - 1u);
}

// 16 bytes of one row starting at byte k (k % 16 == 0), zero past K.
// ALIGNED: row stride and base are 16-byte aligned and the stride is >= the
// 16-rounded K, so a straddling chunk can be read whole and masked. Otherwise
// the row is read as 4-byte words (strides are multiples of 4 by contract).
template <bool ALIGNED>
__device__ __forceinline__ v4i load_chunk(const int8_t* row, int k, int K) {
    v4i r = {0, 0, 0, 0};
    if (k >= K) return r;
    if (ALIGNED) {
        r = *reinterpret_cast<const v4i*>(row + k);
        if (k + 16 > K) {
            r.x = mask_word(r.x, k, K);
            r.y = mask_word(r.y, k + 4, K);
            r.z = mask_word(r.z, k + 8, K);
            r.w = mask_word(r.w, k + 12, K);
        }
        return r;
    }
    const int* p = reinterpret_cast<const int*>(row + k);
    r.x = mask_word(p[0], k, K);
    if (k + 4 < K) r.y = mask_word(p[1], k + 4, K);
    if (k + 8 < K) r.z = mask_word(p[2], k + 8, K);
    if (k + 12 < K) r.w = mask_word(p[3], k + 12, K);
    return r;
}

// One output element of the fused epilogue. mode: 0 store, 1 accumulate,
// 2 raw int32.
__device__ __forceinline__ void store_out(const GemmArgs& a, int m, int n, int acc) {
    if (a.acc32) {
        a.acc32[(size_t)m * a.N + n] = acc;
        return;
    }
    const float p = (float)acc * a.wscale[n];
    float v = fmaf(p, a.ascale[m], a.bias ? a.bias[n] : 0.0f);
    switch (a.act) {
    case 1: v = act_relu(v); break;
    case 2: v = act_gelu_tanh(v); break;
    case 3: v = act_gelu_erf(v); break;
    default: break;
    }
    float* o = a.out + (size_t)m * a.ldo + n;
    if (a.accumulate) v = *o + v;
    *o = v;
}

// XCD-aware tile order (see the file comment).
__device__ __forceinline__ void tile_coords(int bid, int nbm, int nbn, int& tm, int& tn) {
    const int total = nbm * nbn;
    const int x = bid & 7, i = bid >> 3;
    const int per = total >> 3, rem = total & 7;
    const int logical = x * per + (x < rem ? x : rem) + i;
    constexpr int GM = 8;
    const int span = GM * nbn;
    const int group = logical / span;
    const int first = group * GM;
    const int gm = nbm - first < GM ? nbm - first : GM;
    const int in = logical - group * span;
    tm = first + in % gm;
    tn = in / gm;
}

template <int BM, int BN, int BK, int WM, int WN, bool ALIGNED>
__global__ __launch_bounds__(256) void gemm_i8_tiled(GemmArgs a) {
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 16, FN = TN / 16;
    constexpr int SA = BK + 16;                 // padded LDS row, bytes
    constexpr int CPR = BK / 16;                // 16-byte chunks per row
    constexpr int CA = (BM * CPR + 255) / 256;  // chunks per thread, A slab
    constexpr int CB = (BN * CPR + 255) / 256;
    static_assert(WM * WN == 4, "4 waves");
    static_assert(TM % 16 == 0 && TN % 16 == 0 && BK % 64 == 0, "tile shape");

    __shared__ __attribute__((aligned(16))) int8_t smem[2 * (BM + BN) * SA];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;

    int tm, tn;
    tile_coords(blockIdx.x, (a.M + BM - 1) / BM, (a.N + BN - 1) / BN, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int K = a.K;

    // Per-thread slab chunks, fixed across K: chunk c of a slab is row c / CPR,
    // bytes [16*(c % CPR), +16). act: the chunk exists in this slab shape;
    // ok: it also lies inside the matrix (rows past M or N load as zero).
    const int8_t* arow[CA];
    int akc[CA], aoff[CA];
    bool aact[CA], aok[CA];
#pragma unroll
    for (int j = 0; j < CA; j++) {
        const int c = tid + 256 * j;
        const int r = c / CPR;
        akc[j] = (c % CPR) * 16;
        aact[j] = c < BM * CPR;
        aok[j] = aact[j] && m0 + r < a.M;
        arow[j] = a.A + (size_t)(aok[j] ? m0 + r : 0) * a.lda;
        aoff[j] = r * SA + akc[j];
    }
    const int8_t* brow[CB];
    int bkc[CB], boff[CB];
    bool bact[CB], bok[CB];
#pragma unroll
    for (int j = 0; j < CB; j++) {
        const int c = tid + 256 * j;
        const int r = c / CPR;
        bkc[j] = (c % CPR) * 16;
        bact[j] = c < BN * CPR;
        bok[j] = bact[j] && n0 + r < a.N;
        brow[j] = a.B + (size_t)(bok[j] ? n0 + r : 0) * a.ldb;
        boff[j] = BM * SA + r * SA + bkc[j];
    }

    v4i ra[CA], rb[CB];
    auto gload = [&](int k0) {
#pragma unroll
        for (int j = 0; j < CA; j++)
            ra[j] = aok[j] ? load_chunk<ALIGNED>(arow[j], k0 + akc[j], K) : v4i{0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < CB; j++)
            rb[j] = bok[j] ? load_chunk<ALIGNED>(brow[j], k0 + bkc[j], K) : v4i{0, 0, 0, 0};
    };
    auto lstore = [&](int buf) {
        int8_t* s = smem + buf * (BM + BN) * SA;
#pragma unroll
        for (int j = 0; j < CA; j++)
            if (aact[j]) *reinterpret_cast<v4i*>(s + aoff[j]) = ra[j];
#pragma unroll
        for (int j = 0; j < CB; j++)
            if (bact[j]) *reinterpret_cast<v4i*>(s + boff[j]) = rb[j];
    };

    v4i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = v4i{0, 0, 0, 0};

    const int nk = (K + BK - 1) / BK;
    gload(0);
    lstore(0);
    __syncthreads();

    const int arow_l = (wm * TM + (lane & 15)) * SA + (lane >> 4) * 16;
    const int brow_l = BM * SA + (wn * TN + (lane & 15)) * SA + (lane >> 4) * 16;

    for (int kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * BK);
        const int8_t* s = smem + buf * (BM + BN) * SA;
#pragma unroll
        for (int ks = 0; ks < BK / 64; ks++) {
            v4i af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; i++)
                af[i] = *reinterpret_cast<const v4i*>(s + arow_l + i * 16 * SA + ks * 64);
#pragma unroll
            for (int j = 0; j < FN; j++)
                bf[j] = *reinterpret_cast<const v4i*>(s + brow_l + j * 16 * SA + ks * 64);
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++) acc[i][j] = mfma_i8(af[i], bf[j], acc[i][j]);
        }
        if (kt + 1 < nk) lstore(buf ^ 1);
        __syncthreads();
    }

    // epilogue straight from the accumulator layout
    const int mb = m0 + wm * TM + 4 * (lane >> 4);
    const int nb = n0 + wn * TN + (lane & 15);
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int n = nb + j * 16;
            if (n >= a.N) continue;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = mb + i * 16 + r;
                if (m < a.M) store_out(a, m, n, acc[i][j][r]);
            }
        }
}

// ---------------------------------------------------------------- skinny --

template <int FM, int FN, int WAVES, bool ALIGNED>
__global__ __launch_bounds__(WAVES * 64) void gemm_i8_skinny(GemmArgs a, int ksplit,
                                                             int32_t* ws, int32_t* counters) {
    constexpr int TM = FM * 16, TN = FN * 16;
    __shared__ int32_t red[TM * TN];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * TN;
    const int split = blockIdx.y;
    const int K = a.K;

    for (int i = tid; i < TM * TN; i += WAVES * 64) red[i] = 0;

    // k-steps of 64 bytes owned by this block, then by this wave
    const int steps = (K + 63) / 64;
    const int bs0 = (int)((long)steps * split / ksplit), bs1 = (int)((long)steps * (split + 1) / ksplit);
    const int ws0 = bs0 + (int)((long)(bs1 - bs0) * wave / WAVES);
    const int ws1 = bs0 + (int)((long)(bs1 - bs0) * (wave + 1) / WAVES);

    const int r16 = lane & 15, kq = (lane >> 4) * 16;
    const int8_t* arow[FM];
    bool aok[FM];
#pragma unroll
    for (int i = 0; i < FM; i++) {
        aok[i] = i * 16 + r16 < a.M;
        arow[i] = a.A + (size_t)(aok[i] ? i * 16 + r16 : 0) * a.lda;
    }
    const int8_t* brow[FN];
    bool bok[FN];
#pragma unroll
    for (int j = 0; j < FN; j++) {
        bok[j] = n0 + j * 16 + r16 < a.N;
        brow[j] = a.B + (size_t)(bok[j] ? n0 + j * 16 + r16 : 0) * a.ldb;
    }

    v4i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = v4i{0, 0, 0, 0};

    for (int s = ws0; s < ws1; s++) {
        const int k = s * 64 + kq;
        v4i bf[FN], af[FM];
#pragma unroll
        for (int j = 0; j < FN; j++)
            bf[j] = bok[j] ? load_chunk<ALIGNED>(brow[j], k, K) : v4i{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < FM; i++)
            af[i] = aok[i] ? load_chunk<ALIGNED>(arow[i], k, K) : v4i{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) acc[i][j] = mfma_i8(af[i], bf[j], acc[i][j]);
    }

    __syncthreads();
    // exact int32 reduction of the waves' partials
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int mm = i * 16 + 4 * (lane >> 4) + r;
                const int nn = j * 16 + r16;
                if (ws0 < ws1) atomicAdd(&red[mm * TN + nn], acc[i][j][r]);
            }
    __syncthreads();

    if (ksplit > 1) {
        // cross-block split: add this block's slab into the global workspace,
        // then the last block to arrive for this slab finishes it.
        for (int e = tid; e < TM * TN; e += WAVES * 64) {
            const int mm = e / TN, nn = e % TN;
            if (mm < a.M && n0 + nn < a.N) atomicAdd(&ws[(size_t)mm * a.N + n0 + nn], red[e]);
        }
        __threadfence();
        __syncthreads();
        __shared__ int last;
        if (tid == 0) last = atomicAdd(&counters[blockIdx.x], 1) == ksplit - 1;
        __syncthreads();
        if (!last) return;
        __threadfence();
        for (int e = tid; e < TM * TN; e += WAVES * 64) {
            const int mm = e / TN, nn = e % TN;
            if (mm < a.M && n0 + nn < a.N) {
                int32_t* p = &ws[(size_t)mm * a.N + n0 + nn];
                red[e] = atomicExch(p, 0);  // read the sum, leave the workspace zeroed
            }
        }
        if (tid == 0) counters[blockIdx.x] = 0;
        __syncthreads();
    }

    for (int e = tid; e < TM * TN; e += WAVES * 64) {
        const int mm = e / TN, nn = e % TN;
        if (mm < a.M && n0 + nn < a.N) store_out(a, mm, n0 + nn, red[e]);
    }
}

// ---------------------------------------------------------------- launch --

// Grow-only, zero-initialised split-K workspace on the current device. The
// skinny kernel leaves it zeroed after every launch, so one clear suffices.
struct SplitWorkspace {
    int32_t* ws = nullptr;
    int32_t* counters = nullptr;
    size_t ws_elems = 0, n_counters = 0;
    int device = -1;
};
SplitWorkspace g_split[16];

void ensure_split_ws(int dev, size_t elems, size_t counters, hipStream_t st) {
    SplitWorkspace& w = g_split[dev & 15];
    if (w.ws_elems >= elems && w.n_counters >= counters) return;
    VLA_HIP_CHECK(hipStreamSynchronize(st));
    if (w.ws) VLA_HIP_CHECK(hipFree(w.ws));
    if (w.counters) VLA_HIP_CHECK(hipFree(w.counters));
    w.ws_elems = elems > w.ws_elems ? elems : w.ws_elems;
    w.n_counters = counters > w.n_counters ? counters : w.n_counters;
    VLA_HIP_CHECK(hipMalloc(&w.ws, w.ws_elems * sizeof(int32_t)));
    VLA_HIP_CHECK(hipMalloc(&w.counters, w.n_counters * sizeof(int32_t)));
    VLA_HIP_CHECK(hipMemset(w.ws, 0, w.ws_elems * sizeof(int32_t)));
    VLA_HIP_CHECK(hipMemset(w.counters, 0, w.n_counters * sizeof(int32_t)));
    VLA_HIP_CHECK(hipDeviceSynchronize());
}

template <int BM, int BN, int BK, int WM, int WN>
void run_tiled(const GemmArgs& a, bool al, hipStream_t st) {
    const int blocks = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    if (al)
        gemm_i8_tiled<BM, BN, BK, WM, WN, true><<<blocks, 256, 0, st>>>(a);
    else
        gemm_i8_tiled<BM, BN, BK, WM, WN, false><<<blocks, 256, 0, st>>>(a);
    VLA_LAUNCH_CHECK();
}

template <int FM, int FN, int WAVES>
void run_skinny_fm(const GemmArgs& a, bool al, int ksplit, hipStream_t st) {
    const int nb = (a.N + FN * 16 - 1) / (FN * 16);
    int32_t* ws = nullptr;
    int32_t* counters = nullptr;
    if (ksplit > 1) {
        int dev = 0;
        VLA_HIP_CHECK(hipGetDevice(&dev));
        ensure_split_ws(dev, (size_t)a.M * a.N, (size_t)nb, st);
        ws = g_split[dev & 15].ws;
        counters = g_split[dev & 15].counters;
    }
    const dim3 grid(nb, ksplit);
    if (al)
        gemm_i8_skinny<FM, FN, WAVES, true><<<grid, WAVES * 64, 0, st>>>(a, ksplit, ws, counters);
    else
        gemm_i8_skinny<FM, FN, WAVES, false><<<grid, WAVES * 64, 0, st>>>(a, ksplit, ws, counters);
    VLA_LAUNCH_CHECK();
}

template <int FN, int WAVES>
void run_skinny(const GemmArgs& a, bool al, int ksplit, hipStream_t st) {
    const int fm = (a.M + 15) / 16;
    switch (fm) {
    case 1: run_skinny_fm<1, FN, WAVES>(a, al, ksplit, st); break;
    case 2: run_skinny_fm<2, FN, WAVES>(a, al, ksplit, st); break;
    case 3: run_skinny_fm<3, FN, WAVES>(a, al, ksplit, st); break;
    case 4: run_skinny_fm<4, FN, WAVES>(a, al, ksplit, st); break;
    case 5: run_skinny_fm<5, FN, WAVES>(a, al, ksplit, st); break;
    case 6: run_skinny_fm<6, FN, WAVES>(a, al, ksplit, st); break;
    case 7: run_skinny_fm<7, FN, WAVES>(a, al, ksplit, st); break;
    default: run_skinny_fm<8, FN, WAVES>(a, al, ksplit, st); break;
    }
}

constexpr int kCUs = 256;

}  // namespace

void launch_gemm_i8(const GemmArgs& a, hipStream_t st) {
    VLA_REQUIRE(a.M >= 0 && a.N > 0 && a.K > 0, "gemm_i8: need M >= 0, N > 0, K > 0");
    VLA_REQUIRE(a.K <= kMaxI8K, "gemm_i8: K exceeds the int8 accumulator bound INT_MAX/(255*127)");
    VLA_REQUIRE(a.lda >= kpad4(a.K) && a.ldb >= kpad4(a.K) && a.lda % 4 == 0 && a.ldb % 4 == 0,
                "gemm_i8: int8 row strides must be multiples of 4 and >= i8_kpad(K)");
    VLA_REQUIRE(aligned(a.A, 4) && aligned(a.B, 4), "gemm_i8: int8 operands must be 4-byte aligned");
    VLA_REQUIRE(a.acc32 || (a.out && a.wscale && a.ascale && a.ldo >= a.N),
                "gemm_i8: fp32 output needs out, wscale, ascale and ldo >= N");
    VLA_REQUIRE(a.act >= 0 && a.act <= 3, "gemm_i8: unknown activation");
    if (a.M == 0) return;

    const bool al = a.lda % 16 == 0 && a.ldb % 16 == 0 && aligned(a.A, 16) && aligned(a.B, 16);

    if (a.M <= 128) {
        // one block per 16-column slab; split K across blocks until the grid
        // covers the chip about twice (each split adds one int32 pass over the
        // [M, slab] tile through L2 atomics)
        const int nb = (a.N + 15) / 16;
        const int steps = (a.K + 63) / 64;
        int ksplit = 1;
        while (nb * ksplit < 2 * kCUs && steps / (ksplit * 2) >= 4) ksplit *= 2;
        run_skinny<1, 4>(a, al, ksplit, st);
        return;
    }
    const long t256 = (long)((a.M + 255) / 256) * ((a.N + 127) / 128);
    const long t128 = (long)((a.M + 127) / 128) * ((a.N + 127) / 128);
    const long t64 = (long)((a.M + 63) / 64) * ((a.N + 127) / 128);
    if (t256 >= kCUs)
        run_tiled<256, 128, 64, 2, 2>(a, al, st);
    else if (t128 >= kCUs)
        run_tiled<128, 128, 64, 2, 2>(a, al, st);
    else if (t64 >= kCUs)
        run_tiled<64, 128, 64, 2, 2>(a, al, st);
    else
        run_tiled<64, 64, 64, 2, 2>(a, al, st);
}

}  // namespace hip
}  // namespace vla
