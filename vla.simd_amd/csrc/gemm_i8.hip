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
// All kernels use v_mfma_i32_16x16x64_i8: lane l supplies 16 contiguous bytes
// of row (l % 16) at k offset 16*(l / 16) for both operands, so whatever k
// order the unit uses inside one instruction it pairs equal k on both sides.
// Output lane l holds column l % 16, rows 4*(l/16) + r. The tiled and LDS
// kernels pass the weight fragment first, so their accumulators hold the
// output transposed: lane l has output row l % 16 and the 4 consecutive output
// columns 4*(l/16) + r, which it stores as one 16-byte vector.
//
// Kernels
//   gemm_i8_tiled   16-byte aligned rows (every resident layout of this
//                   library). BM x BN block tile, 4 waves in a 2 x 2 grid, K
//                   staged through LDS in BK-byte slabs, double buffered: the
//                   global loads of slab k+2 are issued as soon as slab k+1 is
//                   in LDS, and overlap the MFMAs of slab k+1. The main loop is
//                   branch-free: rows past M or N are clamped to the last row
//                   (their results are never stored) and only the last, partial
//                   K slab is read with byte masks. LDS rows are padded by 16
//                   bytes so the 16 rows one ds_read_b128 touches fall on
//                   distinct bank groups. Workgroups are remapped so each XCD
//                   (the hardware deals workgroup i to XCD i % 8) owns a
//                   contiguous run of tiles, grouped 8 tile-rows deep, which
//                   keeps the A and B panels a run shares in that XCD's L2.
//                   The epilogue stores straight from the accumulators.
//   gemm_i8_lds     long K (> 1024), and large outputs over 512..1024 bytes
//                   of K (128 x 128 tiles), aligned rows. Operand slabs go straight
//                   from global memory into LDS (global_load_lds_dwordx4, no
//                   VGPR staging) with S-1 slabs in flight; LDS rows are
//                   XOR-swizzled by 16-byte chunk instead of padded; the
//                   pipeline barrier waits only for LDS reads (lgkmcnt), not
//                   for the slabs still in flight. Block tiles up to 256 x 256
//                   with 8 waves (WM x WN); same XCD-aware order and epilogue
//                   as gemm_i8_tiled. PF: the LDS reads of the next 64-byte
//                   sub-step and the next slab's loads are interleaved with
//                   the current sub-step's MFMAs (two fragment register sets).
//   gemm_i8_skinny  M <= 128, aligned rows (action chunks, decode rows): one
//                   block owns a 16-column slab of the output and every row; its
//                   waves take interleaved 64-byte k-steps, stream Wq straight
//                   from HBM into MFMA registers (each weight byte is read once),
//                   write their int32 partial tiles to LDS, and each thread sums
//                   one output over the waves before one epilogue. No
//                   cross-block reduction: no global atomics and no device-scope
//                   fences (which write back L2 on a multi-XCD part).
//   gemm_i8_generic any 4-byte aligned strides (the op API accepts the
//                   reference's [seq, i8_kpad(K)] rows, e.g. K = 1027): 64 x 64
//                   tiles, every chunk masked at K.

#include "act.h"
#include "common.h"
#include "rope.h"
#include "rowop.h"

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <type_traits>

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

// The fused epilogue value of one output (before an accumulate).
__device__ __forceinline__ float epi_value(const GemmArgs& a, int m, int n, int acc) {
    const float p = (float)acc * a.wscale[n];
    float v = fmaf(p, a.ascale[m], a.bias ? a.bias[n] : 0.0f);
    switch (a.act) {
    case 1: v = act_relu(v); break;
    case 2: v = act_gelu_tanh(v); break;
    case 3: v = act_gelu_erf(v); break;
    default: break;
    }
    return v;
}

// One output element, straight to global (generic and skinny kernels).
__device__ __forceinline__ void store_out(const GemmArgs& a, int m, int n, int acc) {
    if (a.acc32) {
        a.acc32[(size_t)m * a.N + n] = acc;
        return;
    }
    float v = epi_value(a, m, n, acc);
    float* o = a.out + (size_t)m * a.ldo + n;
    if (a.accumulate) v = *o + v;
    *o = v;
}

typedef float v4f __attribute__((ext_vector_type(4)));

// Orders this wave's LDS accesses: its earlier writes are complete before its
// later reads (other lanes' values), with no block barrier.
__device__ __forceinline__ void wave_lds_sync() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4));  // lgkmcnt(0) only
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
}

// Calls f(std::integral_constant<int, I>) for I = B .. E-1 at compile time, so
// bodies that index register arrays by I keep them in registers however large
// the body (a plain unrolled loop may be left rolled, which forces such arrays
// to scratch).
template <int B, int E>
struct StaticFor {
    template <class F>
    __device__ __forceinline__ static void run(F&& f) {
        f(std::integral_constant<int, B>{});
        StaticFor<B + 1, E>::run(f);
    }
};
template <int E>
struct StaticFor<E, E> {
    template <class F>
    __device__ __forceinline__ static void run(F&&) {}
};

// Weight scales and biases of the 4 consecutive output columns a lane holds
// in each of its FN 16-column blocks (transposed accumulator layout). Loaded
// as 16-byte vectors when the wave's columns are all in range and aligned.
template <int FN>
struct ColOps {
    float ws[FN][4], bs[FN][4];
    __device__ __forceinline__ void load(const GemmArgs& a, int nw, int lane) {
        if (a.acc32) return;
        const int c4 = 4 * (lane >> 4);
        const bool vec = nw + 16 * FN <= a.N && (reinterpret_cast<uintptr_t>(a.wscale) & 15) == 0 &&
                         (!a.bias || (reinterpret_cast<uintptr_t>(a.bias) & 15) == 0);
        if (vec) {
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int n = nw + 16 * j + c4;
                const v4f w = *reinterpret_cast<const v4f*>(a.wscale + n);
                const v4f b = a.bias ? *reinterpret_cast<const v4f*>(a.bias + n) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    ws[j][q] = w[q];
                    bs[j][q] = b[q];
                }
            }
            return;
        }
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int n = nw + 16 * j + c4 + q;
                const int nc = n < a.N ? n : a.N - 1;
                ws[j][q] = a.wscale[nc];
                bs[j][q] = a.bias ? a.bias[nc] : 0.0f;
            }
    }
};

// Epilogue of one wave's TM x TN tile, from accumulators computed transposed
// (mfma_i8(B fragment, A fragment)): lane l of acc[i][j] holds row
// mw + 16 i + (l & 15) and the 4 consecutive columns nw + 16 j + 4 (l >> 4)
// + r. Each lane writes those 4 values to the wave's LDS rows as one 16-byte
// vector, and whole row segments leave as 16-byte stores (NT: non-temporal).
// KIND (0 store, 1 accumulate into out, 2 raw int32 to acc32) and ACT are
// compile-time: the strips are unrolled (the accumulators are registers), and
// a run-time switch inside them would multiply the code many times over and
// leave the epilogue bound by instruction fetch. All row-scale loads are
// issued before the first use, so they share one wait (a later wait would
// also count the output stores in flight).
// KIND 3 is a convolution's residual add + ReLU (out = relu_gt(v +
// resid[m][n])); MX: the wave's max |out| over the rows below M goes to
// *mx_out (max is order-free: the same as a separate pass's block maxima).
template <int TM, int TN, int FM, int FN, int KIND, int ACT, bool NT, bool MX = false>
__device__ __forceinline__ void epilogue_k(const GemmArgs& a, const v4i (&acc)[FM][FN], const ColOps<FN>& co,
                                           int lane, int mw, int nw, float* stage, float* mx_out = nullptr) {
    const int r16 = lane & 15, c4 = 4 * (lane >> 4);
    float mx = 0.0f;
    auto finish = [&]() {
        if constexpr (MX) {
            mx = wave_max_f32(mx);
            if (lane == 0) *mx_out = mx;
        }
    };
    float sa[FM];
    if (KIND != 2) {
#pragma unroll
        for (int i = 0; i < FM; i++) {
            const int m = mw + 16 * i + r16;
            sa[i] = a.ascale[m < a.M ? m : a.M - 1];
        }
    }
    // wave-uniform: whole 16-byte vectors for every column of this wave's tile
    const bool fast = (KIND == 2 ? a.N % 4 == 0 : a.ldo % 4 == 0) && nw + TN <= a.N;
    auto value = [&](int i, int j, int q) {
        const float p = (float)acc[i][j][q] * co.ws[j][q];
        return apply_act<ACT>(fmaf(p, sa[i], co.bs[j][q]));
    };
    if (fast) {
        // per 16-row strip: stage, then row segments of TN * 4 bytes (16 lanes each)
        constexpr int LDW = TN + 4;    // staged row, floats (16-byte multiple)
        constexpr int LPR = TN / 4;    // lanes per row segment
        constexpr int RPI = 64 / LPR;  // rows per store instruction
        StaticFor<0, FM>::run([&](auto ic) {
            constexpr int i = decltype(ic)::value;
#pragma unroll
            for (int j = 0; j < FN; j++) {
                v4f v;
                if (KIND == 2) {
                    v = {__int_as_float(acc[i][j][0]), __int_as_float(acc[i][j][1]),
                         __int_as_float(acc[i][j][2]), __int_as_float(acc[i][j][3])};
                } else {
                    v = {value(i, j, 0), value(i, j, 1), value(i, j, 2), value(i, j, 3)};
                }
                if constexpr (KIND == 3) {
                    const int m = mw + 16 * i + r16;
                    const v4f r = *reinterpret_cast<const v4f*>(a.resid + (size_t)(m < a.M ? m : a.M - 1) * a.ldo +
                                                                 nw + 16 * j + c4);
                    v = {relu_gt(v[0] + r[0]), relu_gt(v[1] + r[1]), relu_gt(v[2] + r[2]), relu_gt(v[3] + r[3])};
                }
                if constexpr (MX) {
                    if (mw + 16 * i + r16 < a.M)
                        mx = fmaxf(fmaxf(mx, fmaxf(fabsf(v[0]), fabsf(v[1]))), fmaxf(fabsf(v[2]), fabsf(v[3])));
                }
                *reinterpret_cast<v4f*>(stage + r16 * LDW + 16 * j + c4) = v;
            }
            wave_lds_sync();
#pragma unroll
            for (int rr = 0; rr < 16; rr += RPI) {
                const int row = rr + lane / LPR, col = (lane % LPR) * 4;
                const int m = mw + 16 * i + row;
                if (m < a.M) {
                    const v4f v = *reinterpret_cast<const v4f*>(stage + row * LDW + col);
                    const int n = nw + col;
                    if (KIND == 2) {
                        *reinterpret_cast<v4f*>(a.acc32 + (size_t)m * a.N + n) = v;
                    } else {
                        float* o = a.out + (size_t)m * a.ldo + n;
                        if (KIND == 1) *reinterpret_cast<v4f*>(o) = *reinterpret_cast<const v4f*>(o) + v;
                        else if (NT) __builtin_nontemporal_store(v, reinterpret_cast<v4f*>(o));
                        else *reinterpret_cast<v4f*>(o) = v;
                    }
                }
            }
            wave_lds_sync();
        });
        finish();
        return;
    }
    // tiles on the N edge, or row strides that are not whole vectors
    StaticFor<0, FM>::run([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        const int m = mw + 16 * i + r16;
        if (m < a.M) {
#pragma unroll
            for (int j = 0; j < FN; j++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int n = nw + 16 * j + c4 + q;
                    if (n < a.N) {
                        if (KIND == 2) {
                            a.acc32[(size_t)m * a.N + n] = acc[i][j][q];
                        } else {
                            float* o = a.out + (size_t)m * a.ldo + n;
                            float v = value(i, j, q);
                            if constexpr (KIND == 3) v = relu_gt(v + a.resid[(size_t)m * a.ldo + n]);
                            if constexpr (MX) mx = fmaxf(mx, fabsf(v));
                            *o = KIND == 1 ? *o + v : v;
                        }
                    }
                }
        }
    });
    finish();
}

// One run-time dispatch to the compile-time epilogue for this launch (CONV:
// only the convolution epilogues, ReLU or residual add + ReLU, with the
// wave's maximum to mx_out).
template <int TM, int TN, int FM, int FN, bool NT, bool CONV = false>
__device__ __forceinline__ void epilogue(const GemmArgs& a, const v4i (&acc)[FM][FN], const ColOps<FN>& co,
                                         int lane, int mw, int nw, float* stage, float* mx_out = nullptr) {
    if constexpr (CONV) {
        if (a.resid) epilogue_k<TM, TN, FM, FN, 3, 0, NT, true>(a, acc, co, lane, mw, nw, stage, mx_out);
        else epilogue_k<TM, TN, FM, FN, 0, 1, NT, true>(a, acc, co, lane, mw, nw, stage, mx_out);
        return;
    }
#define VLA_EPI(KIND, ACT) epilogue_k<TM, TN, FM, FN, KIND, ACT, NT>(a, acc, co, lane, mw, nw, stage)
    if (a.acc32) {
        VLA_EPI(2, 0);
    } else if (a.accumulate) {
        switch (a.act) {
        case 1: VLA_EPI(1, 1); break;
        case 2: VLA_EPI(1, 2); break;
        case 3: VLA_EPI(1, 3); break;
        default: VLA_EPI(1, 0); break;
        }
    } else {
        switch (a.act) {
        case 1: VLA_EPI(0, 1); break;
        case 2: VLA_EPI(0, 2); break;
        case 3: VLA_EPI(0, 3); break;
        default: VLA_EPI(0, 0); break;
        }
    }
#undef VLA_EPI
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

// ----------------------------------------------------------------- tiled --

template <int BM, int BN, int BK>
struct TileCfg {
    static constexpr int TM = BM / 2, TN = BN / 2;
    static constexpr int FM = TM / 16, FN = TN / 16;
    static constexpr int SA = BK + 16;   // padded LDS row, bytes
    static constexpr int CPR = BK / 16;  // 16-byte chunks per row
    static constexpr int CA = BM * CPR / 256, CB = BN * CPR / 256;
    static constexpr int MAIN = 2 * (BM + BN) * SA;
    static constexpr int EPI = 4 * 16 * (TN + 4) * 4;  // staged epilogue, per wave 16 rows
    static constexpr int LDS = MAIN > EPI ? MAIN : EPI;
    static_assert(BM * CPR % 256 == 0 && BN * CPR % 256 == 0, "chunks must split evenly");
    static_assert(TM % 16 == 0 && TN % 16 == 0 && BK % 64 == 0, "tile shape");
};

template <int BM, int BN, int BK>
__global__ __launch_bounds__(256) void gemm_i8_tiled(GemmArgs a) {
    using C = TileCfg<BM, BN, BK>;
    constexpr int TM = C::TM, TN = C::TN, FM = C::FM, FN = C::FN, SA = C::SA, CPR = C::CPR;
    constexpr int CA = C::CA, CB = C::CB;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];

    if (gridDim.y > 1) {  // split K: chunk blockIdx.y of K, raw int32 sums into its workspace slice
        const int k0 = blockIdx.y * a.kchunk;
        a.A += k0;
        a.B += k0;
        a.K = a.K - k0 < a.kchunk ? a.K - k0 : a.kchunk;
        a.acc32 = a.split_ws + (size_t)blockIdx.y * a.M * a.N;
    }

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    int tm, tn;
    tile_coords(blockIdx.x, (a.M + BM - 1) / BM, (a.N + BN - 1) / BN, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int K = a.K;

    // Per-thread slab chunks, fixed across K: chunk c of a slab is row c / CPR,
    // bytes [16*(c % CPR), +16). Rows past the matrix are clamped to its last row.
    const int8_t* arow[CA];
    int aoff[CA];
#pragma unroll
    for (int j = 0; j < CA; j++) {
        const int c = tid + 256 * j, r = c / CPR, kc = (c % CPR) * 16;
        const int m = m0 + r < a.M ? m0 + r : a.M - 1;
        arow[j] = a.A + (size_t)m * a.lda + kc;
        aoff[j] = r * SA + kc;
    }
    const int8_t* brow[CB];
    int boff[CB];
#pragma unroll
    for (int j = 0; j < CB; j++) {
        const int c = tid + 256 * j, r = c / CPR, kc = (c % CPR) * 16;
        const int n = n0 + r < a.N ? n0 + r : a.N - 1;
        brow[j] = a.B + (size_t)n * a.ldb + kc;
        boff[j] = BM * SA + r * SA + kc;
    }

    v4i ra[CA], rb[CB];
    auto gload = [&](int k0) {
#pragma unroll
        for (int j = 0; j < CA; j++) ra[j] = *reinterpret_cast<const v4i*>(arow[j] + k0);
#pragma unroll
        for (int j = 0; j < CB; j++) rb[j] = *reinterpret_cast<const v4i*>(brow[j] + k0);
    };
    auto gload_tail = [&](int k0) {
#pragma unroll
        for (int j = 0; j < CA; j++) {
            const int kc = ((tid + 256 * j) % CPR) * 16;
            ra[j] = load_chunk<true>(arow[j] - kc, k0 + kc, K);
        }
#pragma unroll
        for (int j = 0; j < CB; j++) {
            const int kc = ((tid + 256 * j) % CPR) * 16;
            rb[j] = load_chunk<true>(brow[j] - kc, k0 + kc, K);
        }
    };
    auto lstore = [&](int buf) {
        int8_t* s = smem + buf * (BM + BN) * SA;
#pragma unroll
        for (int j = 0; j < CA; j++) *reinterpret_cast<v4i*>(s + aoff[j]) = ra[j];
#pragma unroll
        for (int j = 0; j < CB; j++) *reinterpret_cast<v4i*>(s + boff[j]) = rb[j];
    };

    v4i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = v4i{0, 0, 0, 0};

    const int arow_l = (wm * TM + (lane & 15)) * SA + (lane >> 4) * 16;
    const int brow_l = BM * SA + (wn * TN + (lane & 15)) * SA + (lane >> 4) * 16;
    auto compute = [&](int buf) {
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
                for (int j = 0; j < FN; j++) acc[i][j] = mfma_i8(bf[j], af[i], acc[i][j]);
        }
    };


    const int nfull = K / BK;            // slabs read without masks
    const int nk = nfull + (K % BK ? 1 : 0);
    if (nfull > 0) gload(0);
    else gload_tail(0);
    lstore(0);
    if (nk > 1) {
        if (1 < nfull) gload(BK);
        else gload_tail(BK);
    }
    __syncthreads();

    for (int kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        compute(buf);
        if (kt + 1 < nk) {
            lstore(buf ^ 1);  // slab kt+1, loaded during the previous compute
            if (kt + 2 < nfull) gload((kt + 2) * BK);
            else if (kt + 2 < nk) gload_tail((kt + 2) * BK);
        }
        __syncthreads();
    }

    // loaded after the loop: held across it they would cost a wave of occupancy
    ColOps<FN> co;
    co.load(a, n0 + wn * TN, lane);
    __syncthreads();  // the staging rows reuse the slab buffers
    epilogue<TM, TN, FM, FN, true>(a, acc, co, lane, m0 + wm * TM, n0 + wn * TN,
                                   reinterpret_cast<float*>(smem) + wave * 16 * (TN + 4));
}

// ------------------------------------------------------ direct-to-LDS --

// 16 zero bytes: the source of every chunk of the last K slab that lies past
// the (16-rounded) row length.
__device__ __attribute__((aligned(16))) int8_t g_zero16[16] = {0};

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their max).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// XOR swizzle of the 16-byte chunks within one LDS row, so the 16 rows one
// ds_read_b128 touches (same logical chunk) land on distinct bank groups.
// Workgroup barrier for the LDS-DMA pipeline. __syncthreads() carries a
// release fence that waits for every outstanding vector load (vmcnt(0)), which
// would drain the slabs in flight; here only this wave's LDS reads must be
// done (lgkmcnt(0)) - the slab being consumed was awaited with wait_vmcnt.
// The empty asm statements keep the compiler from moving memory accesses
// across the barrier.
__device__ __forceinline__ void pipeline_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4));  // lgkmcnt(0) only
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int BK>
__device__ __forceinline__ int swz(int r) {
    return BK == 64 ? (r >> 1) & 3 : r & 7;
}

template <int BM, int BN, int BK, int S, int WM, int WN>
struct LdsCfg {
    static constexpr int NW = WM * WN, NT = 64 * NW;  // waves, threads per block
    static constexpr int TM = BM / WM, TN = BN / WN;
    static constexpr int FM = TM / 16, FN = TN / 16;
    static constexpr int CPR = BK / 16;
    static constexpr int IA = BM * CPR / NT, IB = BN * CPR / NT;  // load instrs per wave per slab
    static constexpr int LPS = IA + IB;
    static constexpr int STAGE = (BM + BN) * BK;
    static constexpr int MAIN = S * STAGE;
    static constexpr int EPI = NW * 16 * (TN + 4) * 4;  // staged epilogue, per wave 16 rows
    static constexpr int LDS = MAIN > EPI ? MAIN : EPI;
    static_assert(BM * CPR % NT == 0 && BN * CPR % NT == 0, "slab chunks must split evenly");
    static_assert(TM % 16 == 0 && TN % 16 == 0, "wave tile");
    static_assert(S >= 2 && (S - 2) * LPS < 64, "pipeline depth");
};

// The block's maximum of its waves' maxima red[0, NW) to omax[blockIdx.x]
// (every wave has written its slot before the barrier).
template <int NW>
__device__ __forceinline__ void conv_block_max(float* omax, const float* red) {
    __syncthreads();
    if (threadIdx.x == 0) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) v = fmaxf(v, red[w]);
        omax[blockIdx.x] = v;
    }
}

// IMPL: A is gathered from an int8 NHWC map as an implicit convolution (the
// GemmArgs cv_ fields): each row's 16-byte chunk of a 128-byte K slab lies in
// one tap, at most one tap past the slab's first (cv_c % 64 == 0), and taps
// outside the image read the zero chunk.
template <int BM, int BN, int BK, int S, int WM, int WN, bool PF, bool CONV = false, bool IMPL = false>
__global__ __launch_bounds__(64 * WM * WN) void gemm_i8_lds(GemmArgs a) {
    // Plain output stores on the 256 x 256 tile (every CU writes its tiles at
    // the same moment; measured faster), non-temporal ones elsewhere.
    constexpr bool NT = BN != 256;
    using C = LdsCfg<BM, BN, BK, S, WM, WN>;
    constexpr int TM = C::TM, TN = C::TN, FM = C::FM, FN = C::FN, CPR = C::CPR, NW = C::NW;
    constexpr int IA = C::IA, IB = C::IB, LPS = C::LPS, STAGE = C::STAGE;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    __shared__ float conv_red[CONV ? NW : 1];  // the convolution epilogue's wave maxima

    const int tid = threadIdx.x;
    // wave index as a scalar, so LDS-DMA destinations are scalar arithmetic
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    int tm, tn;
    tile_coords(blockIdx.x, (a.M + BM - 1) / BM, (a.N + BN - 1) / BN, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int K16 = (a.K + 15) & ~15;
    const int nk = K16 / BK + (K16 % BK ? 1 : 0);  // K slabs

    // Load slots: instruction j of this wave fills LDS chunks [64*slot, +64) of
    // the slab, slot = j*NW + wave; lane l writes chunk 64*slot + l, which holds
    // row q / CPR, logical chunk (q % CPR) ^ swz(row).
    const int8_t* asrc[IA];
    int acb[IA];
    int aiy[IMPL ? IA : 1], aix[IMPL ? IA : 1];  // IMPL: the row's pixel, top-left tap
#pragma unroll
    for (int j = 0; j < IA; j++) {
        const int q = (j * NW + wave) * 64 + lane, r = q / CPR;
        const int c = (q % CPR) ^ swz<BK>(r);
        const int m = m0 + r < a.M ? m0 + r : a.M - 1;
        acb[j] = c * 16;
        if constexpr (IMPL) {
            const int oy = m / a.cv_wo, ox = m - oy * a.cv_wo;
            aiy[j] = oy * a.cv_s - a.cv_p;
            aix[j] = ox * a.cv_s - a.cv_p;
            asrc[j] = a.A;
        } else {
            asrc[j] = a.A + (size_t)m * a.lda + acb[j];
        }
    }
    const int8_t* bsrc[IB];
    int bcb[IB];
#pragma unroll
    for (int j = 0; j < IB; j++) {
        const int q = (j * NW + wave) * 64 + lane, r = q / CPR;
        const int c = (q % CPR) ^ swz<BK>(r);
        const int n = n0 + r < a.N ? n0 + r : a.N - 1;
        bcb[j] = c * 16;
        bsrc[j] = a.B + (size_t)n * a.ldb + bcb[j];
    }

    typedef __attribute__((address_space(1))) const void* gptr;
    typedef __attribute__((address_space(3))) void* lptr;
    // Slab kt into stage kt % S. A slab index past the last one reloads the
    // last slab (PF issues unconditionally; such a stage is never read again).
    auto issue = [&](int kt) {
        const int k0 = (kt < nk ? kt : nk - 1) * BK;
        int8_t* st = smem + (kt % S) * STAGE;
        const bool full = k0 + BK <= K16;
        if constexpr (IMPL) {
            // the slab's first tap (ky0, kx0) at channel ci0, and the tap after it
            const int tap0 = k0 / a.cv_c, ci0 = k0 - tap0 * a.cv_c;
            const int ky0 = tap0 / a.cv_k, kx0 = tap0 - ky0 * a.cv_k;
            const int ky1 = kx0 + 1 == a.cv_k ? ky0 + 1 : ky0, kx1 = kx0 + 1 == a.cv_k ? 0 : kx0 + 1;
#pragma unroll
            for (int j = 0; j < IA; j++) {
                int ci = ci0 + acb[j], ky = ky0, kx = kx0;
                if (ci >= a.cv_c) {
                    ci -= a.cv_c;
                    ky = ky1;
                    kx = kx1;
                }
                const int iy = aiy[j] + ky, ix = aix[j] + kx;
                const bool in = k0 + acb[j] < K16 && iy >= 0 && iy < a.cv_h && ix >= 0 && ix < a.cv_w;
                const int8_t* p = in ? asrc[j] + ((size_t)iy * a.cv_w + ix) * a.cv_c + ci : g_zero16;
                __builtin_amdgcn_global_load_lds((gptr)p, (lptr)(st + (j * NW + wave) * 1024), 16, 0, 0);
            }
        } else {
#pragma unroll
            for (int j = 0; j < IA; j++) {
                const int8_t* p = full || k0 + acb[j] < K16 ? asrc[j] + k0 : g_zero16;
                __builtin_amdgcn_global_load_lds((gptr)p, (lptr)(st + (j * NW + wave) * 1024), 16, 0, 0);
            }
        }
#pragma unroll
        for (int j = 0; j < IB; j++) {
            const int8_t* p = full || k0 + bcb[j] < K16 ? bsrc[j] + k0 : g_zero16;
            __builtin_amdgcn_global_load_lds((gptr)p, (lptr)(st + BM * BK + (j * NW + wave) * 1024), 16, 0, 0);
        }
    };

    v4i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = v4i{0, 0, 0, 0};
    ColOps<FN> co;  // the plain loop has registers to spare: loaded now, latency hidden
    if constexpr (!PF) co.load(a, n0 + wn * TN, lane);

    const int r16 = lane & 15, cq = lane >> 4;
    const int sz = swz<BK>(r16);  // swz depends on the row's low bits only
    const int arow_l = (wm * TM + r16) * BK;
    const int brow_l = BM * BK + (wn * TN + r16) * BK;


#pragma unroll
    for (int s = 0; s < S - 1; s++)
        if (s < nk) issue(s);

    // Slab kt has landed for this wave once at most the later slabs' loads
    // (slabs kt+1 .. kt+S-2 that exist) are pending.
    auto wait_slab = [&](int kt) {
        const int later = nk - 1 - kt < S - 2 ? nk - 1 - kt : S - 2;
        if (later >= S - 2) wait_vmcnt<(S - 2) * LPS>();
        else if (S > 3 && later == 1) wait_vmcnt<(S > 3 ? LPS : 0)>();
        else if (S > 4 && later == 2) wait_vmcnt<(S > 4 ? 2 * LPS : 0)>();
        else wait_vmcnt<0>();
    };

    if constexpr (PF) {
        // Fragment pipeline: the LDS reads of the next 64-byte sub-step are
        // issued between the MFMAs of the current one (two register sets), so
        // a wave waits for LDS once per sub-step at most and usually not at
        // all. The slab barrier sits between a slab's two sub-steps: by then
        // this wave's reads of slab kt are complete (the barrier waits for
        // them), so slab kt's stage can be refilled with slab kt+S.
        static_assert(BK == 128, "two 64-byte sub-steps per slab");
        v4i fa0[FM], fb0[FN], fa1[FM], fb1[FN];
        auto frag = [&](const int8_t* st, int ks, v4i(&af)[FM], v4i(&bf)[FN]) {
            const int co = 16 * ((ks * 4 + cq) ^ sz);
#pragma unroll
            for (int i = 0; i < FM; i++) af[i] = *reinterpret_cast<const v4i*>(st + arow_l + i * 16 * BK + co);
#pragma unroll
            for (int j = 0; j < FN; j++) bf[j] = *reinterpret_cast<const v4i*>(st + brow_l + j * 16 * BK + co);
        };
        auto mma = [&](const v4i(&af)[FM], const v4i(&bf)[FN]) {
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++) acc[i][j] = mfma_i8(bf[j], af[i], acc[i][j]);
        };
        // one LDS read after each of the first FM+FN MFMAs, then the rest
        auto interleave = [&]() {
            StaticFor<0, FM + FN>::run([&](auto) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            });
            __builtin_amdgcn_sched_group_barrier(0x008, FM * FN - (FM + FN), 0);
        };
        // after the barrier: the slab loads, then the LDS reads, each behind
        // an MFMA, so the matrix pipe restarts as soon as the barrier opens
        static_assert(FM * FN >= LPS + FM + FN, "not enough MFMAs to cover the loads");
        auto interleave_dma = [&]() {
            StaticFor<0, LPS>::run([&](auto) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            });
            StaticFor<0, FM + FN>::run([&](auto) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            });
            __builtin_amdgcn_sched_group_barrier(0x008, FM * FN - (LPS + FM + FN), 0);
        };
        wait_slab(0);
        pipeline_barrier();
        if (S - 1 < nk) issue(S - 1);
        frag(smem, 0, fa0, fb0);
        for (int kt = 0; kt < nk; kt++) {
            frag(smem + (kt % S) * STAGE, 1, fa1, fb1);
            mma(fa0, fb0);
            interleave();
            // every MFMA of the first sub-step is issued before the barrier,
            // which then finds this wave's reads of slab kt long complete
            __builtin_amdgcn_sched_barrier(0);
            // branch-free from here to the MFMAs, so the reads of the next
            // slab interleave with them (the last iteration re-reads its own
            // slab, unused)
            wait_slab(kt + 1);
            pipeline_barrier();
            issue(kt + S);
            const int nxt = kt + 1 < nk ? kt + 1 : kt;
            frag(smem + (nxt % S) * STAGE, 0, fa0, fb0);
            mma(fa1, fb1);
            interleave_dma();
        }
        wait_vmcnt<0>();  // the reloads past the last slab land before LDS is reused or released
        __syncthreads();  // the staging rows reuse the slab buffers
        co.load(a, n0 + wn * TN, lane);  // after the loop: no registers to spare during it
        epilogue<TM, TN, FM, FN, NT, CONV>(a, acc, co, lane, m0 + wm * TM, n0 + wn * TN,
                                           reinterpret_cast<float*>(smem) + wave * 16 * (TN + 4), conv_red + wave);
        if constexpr (CONV) conv_block_max<NW>(a.omax, conv_red);
        return;
    }

    for (int kt = 0; kt < nk; kt++) {
        wait_slab(kt);
        pipeline_barrier();  // every wave's part of slab kt is in LDS; slab kt-1 is consumed
        if (kt + S - 1 < nk) issue(kt + S - 1);
        const int8_t* st = smem + (kt % S) * STAGE;
#pragma unroll
        for (int ks = 0; ks < BK / 64; ks++) {
            const int co = 16 * ((ks * 4 + cq) ^ sz);
            v4i af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; i++) af[i] = *reinterpret_cast<const v4i*>(st + arow_l + i * 16 * BK + co);
#pragma unroll
            for (int j = 0; j < FN; j++) bf[j] = *reinterpret_cast<const v4i*>(st + brow_l + j * 16 * BK + co);
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++) acc[i][j] = mfma_i8(bf[j], af[i], acc[i][j]);
        }
    }
    __syncthreads();  // the staging rows reuse the slab buffers
    epilogue<TM, TN, FM, FN, NT, CONV>(a, acc, co, lane, m0 + wm * TM, n0 + wn * TN,
                                       reinterpret_cast<float*>(smem) + wave * 16 * (TN + 4), conv_red + wave);
    if constexpr (CONV) conv_block_max<NW>(a.omax, conv_red);
}

// ---------------------------------------------------------------- skinny --

// ROPE: blocks below a.rope_cols own 8 rotation pairs of one head instead of
// 16 consecutive columns - lane c < 8 column 8 k + c of the head, lane c >= 8
// its partner 8 k + c - 8 + half (k = the block's index within the head) -
// so the epilogue rotates each output with its partner's value, summed from
// the same block's partial tiles.
// FN: column groups of 16 per block; each A fragment a wave loads feeds FN
// MFMAs from registers, so a block of 16 x FN columns reads its rows of A once
// (the rotating epilogue keeps FN = 1).
// bx: the block's column block (blockIdx.x, or its index within one of the
// two products of gemm_i8_skinny_pair); part: the block's LDS for the waves'
// partial int32 tiles in MFMA lane order, [wave][t][r][lane].
// IMPL: A is gathered from an int8 NHWC map as an implicit convolution (the
// GemmArgs cv_ fields, cv_c % 64 == 0, so each 64-byte step lies in one tap);
// rows whose tap falls outside the image read the zero chunk.
template <int FM, int WAVES, bool ROPE, int FN, bool IMPL = false>
__device__ __forceinline__ void skinny_block(GemmArgs a, const int bx, int32_t* part) {
    static_assert(FM * FN * WAVES <= 64, "partial tiles must fit in 64 KiB of LDS");
    static_assert(!ROPE || FN == 1, "the rotating epilogue owns 16 columns per block");
    constexpr int FT = FM * FN;  // 16 x 16 tiles per wave, tile t = i * FN + j

    if (gridDim.y > 1) {  // split K: chunk blockIdx.y of K (a multiple of 128 bytes), raw int32 sums
        const int k0 = blockIdx.y * a.kchunk;
        a.A += a.a_panel ? (size_t)(k0 / 64) * panel_rows(a.M) * 64 : (size_t)k0;
        a.B += k0;
        a.K = a.K - k0 < a.kchunk ? a.K - k0 : a.kchunk;
        a.acc32 = a.split_ws + (size_t)blockIdx.y * a.M * a.N;
    }

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int n0 = bx * 16 * FN;
    const int K = a.K;
    // row group blockIdx.z: 16-row fragments f0 .. f0 + FM - 1 (fragments past
    // the last one repeat it; their rows are >= M and never stored)
    const int f0 = blockIdx.z * FM, nfrag = (a.M + 15) >> 4;

    // A fragment i of k-step s is at arow[i] + s * astep: row-major rows
    // (clamped to the last row), or the panel layout, where the fragment's 16
    // rows x 64 bytes are contiguous (rows past M are padding, never stored)
    const int r16 = lane & 15, kq = (lane >> 4) * 16;
    const size_t astep = a.a_panel ? (size_t)panel_rows(a.M) * 64 : 64;
    const int8_t* arow[FM];
    int aiy[IMPL ? FM : 1], aix[IMPL ? FM : 1];  // IMPL: the row's pixel, top-left tap
#pragma unroll
    for (int i = 0; i < FM; i++) {
        const int row = (f0 + i < nfrag ? f0 + i : nfrag - 1) * 16 + r16;
        const int m = row < a.M ? row : a.M - 1;
        if constexpr (IMPL) {
            const int oy = m / a.cv_wo, ox = m - oy * a.cv_wo;
            aiy[i] = oy * a.cv_s - a.cv_p;
            aix[i] = ox * a.cv_s - a.cv_p;
            arow[i] = a.A + kq;
        } else {
            arow[i] = a.a_panel ? a.A + (size_t)row * 64 + kq : a.A + (size_t)m * a.lda + kq;
        }
    }
    // output column of block lane c (16 consecutive columns, or ROPE pairs)
    const bool rotb = ROPE && n0 < a.rope_cols;
    auto col = [&](int c) {
        if (!rotb) return n0 + c;
        const int hb = a.rope_hd / 16, head = bx / hb, k = bx - head * hb;
        return head * a.rope_hd + 8 * k + (c & 7) + (c < 8 ? 0 : a.rope_hd / 2);
    };
    const int8_t* brow[FN];
#pragma unroll
    for (int j = 0; j < FN; j++) {
        const int nr = col(16 * j + r16);
        brow[j] = a.B + (size_t)(nr < a.N ? nr : a.N - 1) * a.ldb + kq;
    }

    // The outputs this thread stores after the reduction (element e of the
    // FM x 4 x 64 lane-major tile), and their epilogue operands, fetched now so
    // their latency hides under the main loop rather than after the barrier.
    constexpr int NT = WAVES * 64, EPT = (FT * 256 + NT - 1) / NT;
    float esa[EPT], ews[EPT], eb[EPT], eold[EPT];
    // ROPE: the partner column's scale and bias, this output's (cos, sin)
    float pws[ROPE ? EPT : 1], pb[ROPE ? EPT : 1];
    double rc[ROPE ? EPT : 1], rs[ROPE ? EPT : 1];
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        const int e = tid + j * NT;
        const int l = e & 63, r = (e >> 6) & 3, i = (e >> 8) / FN, jn = (e >> 8) % FN;
        int mm = 16 * (f0 + i) + 4 * (l >> 4) + r, nn = col(16 * jn + (l & 15));
        const bool ok = e < FT * 256 && mm < a.M && nn < a.N;
        mm = ok ? mm : 0;
        nn = ok ? nn : 0;
        esa[j] = ews[j] = eb[j] = eold[j] = 0.0f;
        if (!a.acc32) {
            esa[j] = a.ascale[mm];
            ews[j] = a.wscale[nn];
            eb[j] = a.bias ? a.bias[nn] : 0.0f;
            if (a.accumulate && ok) eold[j] = a.out[(size_t)mm * a.ldo + nn];
            if (a.resid && ok) eold[j] = a.resid[(size_t)mm * a.ldo + nn];  // the convolution's residual
        }
        if constexpr (ROPE) {
            pws[j] = pb[j] = 0.0f;
            rc[j] = rs[j] = 0.0;
            if (rotb && ok) {
                const int np = col((l & 15) ^ 8), half = a.rope_hd / 2;
                pws[j] = a.wscale[np];
                pb[j] = a.bias ? a.bias[np] : 0.0f;
                const double* t = a.rope_cs + ((size_t)mm * half + nn % a.rope_hd % half) * 2;
                rc[j] = t[0];
                rs[j] = t[1];
            }
        }
    }

    v4i acc[FT];
#pragma unroll
    for (int t = 0; t < FT; t++) acc[t] = v4i{0, 0, 0, 0};

    // This wave's 64-byte k-steps are wave, wave + WAVES, ... < full, rotated
    // by a per-block offset: every block reads all of A, and without the
    // rotation the blocks of an XCD would all read the same A lines at the
    // same moment and queue on the same L2 channels (the int32 sums do not
    // depend on the order). The loads run P steps ahead of the MFMAs in a
    // register ring.
    const int full = K / 64;  // 64-byte steps read without masks
    constexpr int FL = FM + FN - 1;  // fragments per step beyond one weight fragment
    constexpr int P = (FL <= 3 || (FL == 4 && WAVES < 16)) ? 4 : 3;  // within the VGPR budget
    // blocks i, i + 8, i + 16, ... share an XCD; (WAVES + 1) is odd, so their
    // offsets differ for up to `full` blocks when full is a power of two
    const int rot = full > 0 ? (int)(((unsigned)bx >> 3) * (WAVES + 1) % (unsigned)full) : 0;
    v4i ra[P][FM], rb[P][FN];
    auto load = [&](int p, int k) {
        int step = wave + k * WAVES + rot;
        step = step < full ? step : step - full;
#pragma unroll
        for (int j = 0; j < FN; j++) rb[p][j] = *reinterpret_cast<const v4i*>(brow[j] + step * 64);
        if constexpr (IMPL) {
            // the step's tap and channel (wave-uniform), then each row's pixel
            const int kk = step * 64, tap = kk / a.cv_c, ci = kk - tap * a.cv_c;
            const int ky = tap / a.cv_k, kx = tap - ky * a.cv_k;
#pragma unroll
            for (int i = 0; i < FM; i++) {
                const int iy = aiy[i] + ky, ix = aix[i] + kx;
                const bool in = iy >= 0 && iy < a.cv_h && ix >= 0 && ix < a.cv_w;
                const int8_t* src = in ? arow[i] + ((size_t)iy * a.cv_w + ix) * a.cv_c + ci : g_zero16;
                ra[p][i] = *reinterpret_cast<const v4i*>(src);
            }
        } else {
            const size_t aoff = (size_t)step * astep;
#pragma unroll
            for (int i = 0; i < FM; i++) ra[p][i] = *reinterpret_cast<const v4i*>(arow[i] + aoff);
        }
    };
    const int nst = wave < full ? (full - wave + WAVES - 1) / WAVES : 0;
    StaticFor<0, P>::run([&](auto pc) {
        constexpr int p = decltype(pc)::value;
        if (p < nst) load(p, p);
    });
    for (int k0 = 0; k0 < nst; k0 += P) {
        StaticFor<0, P>::run([&](auto pc) {
            constexpr int p = decltype(pc)::value;
            const int k = k0 + p;
            if (k < nst) {
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++) acc[i * FN + j] = mfma_i8(ra[p][i], rb[p][j], acc[i * FN + j]);
                if (k + P < nst) load(p, k + P);
            }
        });
    }
    if (K % 64 && wave == full % WAVES) {
        const int k = full * 64 + kq;
        v4i b0[FN];
#pragma unroll
        for (int j = 0; j < FN; j++) b0[j] = load_chunk<true>(brow[j] - kq, k, K);  // zero past K: A bytes there add nothing
#pragma unroll
        for (int i = 0; i < FM; i++) {
            const v4i av = a.a_panel ? *reinterpret_cast<const v4i*>(arow[i] + (size_t)full * astep)
                                     : load_chunk<true>(arow[i] - kq, k, K);
#pragma unroll
            for (int j = 0; j < FN; j++) acc[i * FN + j] = mfma_i8(av, b0[j], acc[i * FN + j]);
        }
    }

    // partial tiles to LDS (no two waves share an address), then each thread
    // sums one element over the waves (exact int32) and stores it
#pragma unroll
    for (int t = 0; t < FT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) part[((wave * FT + t) * 4 + r) * 64 + lane] = acc[t][r];
    __syncthreads();
    float mx = 0.0f;  // the convolution epilogue's max |out| (a.omax)
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        const int e = tid + j * NT;
        if (e >= FT * 256) break;
        int32_t v = 0;
#pragma unroll
        for (int w = 0; w < WAVES; w++) v += part[w * FT * 256 + e];
        const int l = e & 63, r = (e >> 6) & 3, i = (e >> 8) / FN, jn = (e >> 8) % FN;
        const int mm = 16 * (f0 + i) + 4 * (l >> 4) + r, nn = col(16 * jn + (l & 15));
        if (mm >= a.M || nn >= a.N) continue;
        if (a.acc32) {
            a.acc32[(size_t)mm * a.N + nn] = v;
            continue;
        }
        const float p = (float)v * ews[j];
        float o = fmaf(p, esa[j], eb[j]);
        if constexpr (ROPE) {
            if (rotb) {  // act 0, no accumulate (checked by the launcher)
                int32_t vp = 0;
#pragma unroll
                for (int w = 0; w < WAVES; w++) vp += part[w * FT * 256 + (e ^ 8)];
                const float op = fmaf((float)vp * pws[j], esa[j], pb[j]);
                a.out[(size_t)mm * a.ldo + nn] = (l & 8) ? rope_hi(op, o, rc[j], rs[j]) : rope_lo(o, op, rc[j], rs[j]);
                continue;
            }
        }
        if (a.resid) {
            o = relu_gt(o + eold[j]);
        } else {
            switch (a.act) {
            case 1: o = act_relu(o); break;
            case 2: o = act_gelu_tanh(o); break;
            case 3: o = act_gelu_erf(o); break;
            default: break;
            }
        }
        mx = fmaxf(mx, fabsf(o));
        a.out[(size_t)mm * a.ldo + nn] = a.accumulate ? eold[j] + o : o;
    }
    if (a.omax) {  // the block's maximum (part is free once every thread has summed)
        mx = wave_max_f32(mx);
        __syncthreads();
        float* red = reinterpret_cast<float*>(part);
        if (lane == 0) red[wave] = mx;
        __syncthreads();
        if (tid == 0) {
            float v = 0.0f;
            for (int w = 0; w < WAVES; w++) v = fmaxf(v, red[w]);
            a.omax[blockIdx.z * gridDim.x + blockIdx.x] = v;
        }
    }
}

template <int FM, int WAVES, bool ROPE = false, int FN = 1, bool IMPL = false>
__global__ __launch_bounds__(WAVES * 64) void gemm_i8_skinny(GemmArgs a) {
    __shared__ int32_t part[WAVES * FM * FN * 256];
    skinny_block<FM, WAVES, ROPE, FN, IMPL>(a, blockIdx.x, part);
}

// Two independent products over the same rows in one launch (ACT's q | k
// from x + pos beside v from x): column blocks below nb1 are a1's, the rest
// a2's, with one row-group count; each block runs exactly the code and sums
// of its product's own launch, so the outputs are the same bits.
template <int FM, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void gemm_i8_skinny_pair(GemmArgs a1, GemmArgs a2, int nb1) {
    __shared__ int32_t part[WAVES * FM * 256];
    if ((int)blockIdx.x < nb1) skinny_block<FM, WAVES, false, 1>(a1, blockIdx.x, part);
    else skinny_block<FM, WAVES, false, 1>(a2, blockIdx.x - nb1, part);
}

// ------------------------------------------------------------------ gemv --

// One or two rows (decode rows) over a long K: an MFMA fragment would be 16
// rows, 14 or 15 of them padding that every block reads, so these rows take
// dot products instead.
// L lanes share one weight row (output column): lane g of the group takes the
// 16-byte chunks g, g + L, ... of the row and the same chunks of each
// activation row, sums them with v_dot4_i32_i8 (exact int32), and the group's
// sums meet by lane shuffles (exact) before lane 0 applies the epilogue
// (store_out: epi_value, the expression of every other kernel). Weight bytes
// past K are masked to zero, so activation bytes there add nothing.
template <int MV, int L>
__global__ __launch_bounds__(256) void gemm_i8_gemv(GemmArgs a) {
    constexpr int RPW = 64 / L, U = 4;  // rows per wave; chunks in flight per lane
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = (blockIdx.x * 4 + wave) * RPW + lane / L, gl = lane % L;
    const int K = a.K, nch = (K + 15) >> 4;
    const bool nok = n < a.N;
    const int8_t* brow = a.B + (size_t)(nok ? n : a.N - 1) * a.ldb;
    const size_t pstep = (size_t)panel_rows(a.M) * 64;
    int acc[MV];
#pragma unroll
    for (int m = 0; m < MV; m++) acc[m] = 0;
    for (int c0 = gl; c0 < nch; c0 += U * L) {
        v4i w[U], x[U][MV];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int c = c0 + u * L, k = c * 16;
            w[u] = load_chunk<true>(brow, k, K);
#pragma unroll
            for (int m = 0; m < MV; m++) {
                const int8_t* xp = a.a_panel ? a.A + (size_t)(k >> 6) * pstep + m * 64 + (k & 63)
                                             : a.A + (size_t)m * a.lda + k;
                x[u][m] = c < nch ? *reinterpret_cast<const v4i*>(xp) : v4i{0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int m = 0; m < MV; m++) {
                acc[m] = __builtin_amdgcn_sdot4(w[u].x, x[u][m].x, acc[m], false);
                acc[m] = __builtin_amdgcn_sdot4(w[u].y, x[u][m].y, acc[m], false);
                acc[m] = __builtin_amdgcn_sdot4(w[u].z, x[u][m].z, acc[m], false);
                acc[m] = __builtin_amdgcn_sdot4(w[u].w, x[u][m].w, acc[m], false);
            }
    }
#pragma unroll
    for (int off = L / 2; off > 0; off >>= 1)
#pragma unroll
        for (int m = 0; m < MV; m++) acc[m] += __shfl_xor(acc[m], off);
    if (gl == 0 && nok)
#pragma unroll
        for (int m = 0; m < MV; m++)
            if (m < a.M) store_out(a, m, n, acc[m]);
}

// ------------------------------------------------------- row op + skinny --

// Rows the fused row-op GEMM below computes: M rounded up to 16, 32, 64 or 128
// (16 x its FM template value); the LDS it needs for K: the quantized panel
// [K64 / 64][rows][64] or, after the product, the 16 waves' int32 partial
// tiles (16 x FM KiB), whichever is larger, then the rows' scales.
__host__ __device__ inline int rowop_fm(int M) { return M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : 8; }
__host__ __device__ inline int rowop_lds_main(int fm, int K) {
    const int panel = 16 * fm * ((K + 63) & ~63), part = 16 * fm * 1024;
    return panel > part ? panel : part;
}
constexpr int kRowopMaxLds = 160 * 1024;

// gemm_i8_skinny with its activations built in the block (launch_gemm_i8_rowop):
// each block first loads its weight chunks (16 output columns; the 16 waves
// take interleaved 64-byte k-steps, at most two each for K <= 2048), so their
// latency hides under the row op; then wave w applies the row op to rows
// w, w + 16, ... (RB rows in flight, their reductions interleaved), quantizes
// each row exactly as rowq_kernel does (same functions, same order) into the
// LDS panel, and keeps its scale in LDS. After a barrier each wave multiplies
// its k-steps of the panel by its weight chunks; the partial tiles reuse the
// panel's LDS and are summed as in gemm_i8_skinny. Panel rows past M and
// panel bytes past K are never written: the former only reach discarded
// outputs, the latter meet weight bytes masked to zero. With r.q set, the
// first column block of each row group also writes its quantized rows
// row-major (stride r.ldq, bytes [K, r.ldq) zero) and their scales to r.qs:
// the caller-owned scratch of the op API, filled as the quantizer fills it.
template <int OP, int NV, int FM>
__global__ __launch_bounds__(1024) void gemm_i8_rowop(RowQArgs r, GemmArgs a) {
    constexpr int WAVES = 16, NT = WAVES * 64, MP = 16 * FM;
    // rows in flight per wave: at most 4, and 16 float4 per lane, within 128
    // VGPRs. (LayerNorm's double statistics spill at this thread count: op 1
    // stays on rowq_kernel + gemm_i8_skinny.)
    static_assert(OP != 1, "LayerNorm is not fused");
    constexpr int RB = FM < (16 / NV > 4 ? 4 : 16 / NV) ? FM : (16 / NV > 4 ? 4 : 16 / NV);
    static_assert(FM % RB == 0, "row batches must tile the wave's rows");
    extern __shared__ __attribute__((aligned(16))) int8_t lds[];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = a.M, K = a.K, n0 = blockIdx.x * 16;
    const int m0 = blockIdx.y * MP;  // row group: rows m0 .. m0 + MP - 1 (local rows in LDS)
    const int ns = (K + 63) >> 6, full = K >> 6;
    int8_t* panel = lds;
    int32_t* part = reinterpret_cast<int32_t*>(lds);
    float* sa = reinterpret_cast<float*>(lds + rowop_lds_main(FM, K));

    // this wave's weight chunks: k-steps wave and wave + 16 (the last one
    // masked to zero past K)
    const int r16 = lane & 15, kq = (lane >> 4) * 16;
    const int n = n0 + r16 < a.N ? n0 + r16 : a.N - 1;
    const int8_t* brow = a.B + (size_t)n * a.ldb;
    v4i rb[2];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const int step = wave + WAVES * s;
        rb[s] = v4i{0, 0, 0, 0};
        if (step < full) rb[s] = *reinterpret_cast<const v4i*>(brow + step * 64 + kq);
        else if (step < ns) rb[s] = load_chunk<true>(brow, step * 64 + kq, K);
    }

    // epilogue operands of the outputs this thread stores (as gemm_i8_skinny)
    constexpr int EPT = (FM * 256 + NT - 1) / NT;
    float ews[EPT], eb[EPT], eold[EPT];
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        const int e = tid + j * NT;
        const int l = e & 63, rr = (e >> 6) & 3, i = e >> 8;
        int mm = m0 + 16 * i + 4 * (l >> 4) + rr, nn = n0 + (l & 15);
        const bool ok = e < FM * 256 && mm < M && nn < a.N;
        mm = ok ? mm : 0;
        nn = ok ? nn : 0;
        ews[j] = a.wscale[nn];
        eb[j] = a.bias ? a.bias[nn] : 0.0f;
        eold[j] = a.accumulate && ok ? a.out[(size_t)mm * a.ldo + nn] : 0.0f;
    }

    // row op + quantize into the panel
    StaticFor<0, FM / RB>::run([&](auto bc) {
        constexpr int j0 = decltype(bc)::value * RB;
        float4 y[RB][NV];
        int row[RB];
        RowStat st[RB];
        float am[RB];
        StaticFor<0, RB>::run([&](auto jc) {
            constexpr int jj = decltype(jc)::value;
            row[jj] = wave + WAVES * (j0 + jj);
            const int rc = m0 + row[jj] < M ? m0 + row[jj] : M - 1;  // rows past M: a duplicate, never stored
            rowop_load<NV>(y[jj], r.x + (size_t)rc * r.ldx, K, lane);
        });
        StaticFor<0, RB>::run([&](auto jc) {
            constexpr int jj = decltype(jc)::value;
            st[jj] = rowop_stat<OP, NV>(y[jj], r.eps, K, lane);
        });
        StaticFor<0, RB>::run([&](auto jc) {
            constexpr int jj = decltype(jc)::value;
            const int rc = m0 + row[jj] < M ? m0 + row[jj] : M - 1;
            rowop_finish<OP, NV>(y[jj], st[jj], OP == 3 ? r.u + (size_t)rc * r.ldu : nullptr, r.w, r.b, K,
                                 lane);
            am[jj] = rowop_amax<NV>(y[jj], K, lane);
        });
        StaticFor<0, RB>::run([&](auto jc) {
            constexpr int jj = decltype(jc)::value;
            am[jj] = wave_max_f32(am[jj]);
        });
        StaticFor<0, RB>::run([&](auto jc) {
            constexpr int jj = decltype(jc)::value;
            if (m0 + row[jj] < M) {
                const float s = row_scale(am[jj]);
                const float inv = 1.0f / s;
                if (lane == 0) sa[row[jj]] = s;
                int8_t* qr = panel + row[jj] * 64;
#pragma unroll
                for (int i = 0; i < NV; i++) {
                    const int k = 4 * lane + 256 * i;
                    if (k < K) *reinterpret_cast<uint32_t*>(qr + (k >> 6) * (MP * 64) + (k & 63)) = q8x4(y[jj][i], inv);
                }
                if (r.q && blockIdx.x == 0) {  // block-uniform
                    int8_t* gq = r.q + (size_t)(m0 + row[jj]) * r.ldq;
#pragma unroll
                    for (int i = 0; i < NV; i++) {
                        const int k = 4 * lane + 256 * i;
                        if (k < K) *reinterpret_cast<uint32_t*>(gq + k) = q8x4(y[jj][i], inv);
                    }
                    for (int k = K + 4 * lane; k < r.ldq; k += 256) *reinterpret_cast<uint32_t*>(gq + k) = 0u;
                    if (lane == 0) r.qs[m0 + row[jj]] = s;
                }
            }
        });
    });
    __syncthreads();

    v4i acc[FM];
#pragma unroll
    for (int i = 0; i < FM; i++) acc[i] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const int step = wave + WAVES * s;
        if (step < ns) {
            const int8_t* ap = panel + step * (MP * 64) + r16 * 64 + kq;
            v4i av[FM];
#pragma unroll
            for (int i = 0; i < FM; i++) av[i] = *reinterpret_cast<const v4i*>(ap + i * 1024);
#pragma unroll
            for (int i = 0; i < FM; i++) acc[i] = mfma_i8(av[i], rb[s], acc[i]);
        }
    }
    __syncthreads();  // the panel's LDS becomes the partial tiles
    const int nw = ns < WAVES ? ns : WAVES;  // waves that hold a k-step
    if (wave < nw) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int q = 0; q < 4; q++) part[((wave * FM + i) * 4 + q) * 64 + lane] = acc[i][q];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        const int e = tid + j * NT;
        if (e >= FM * 256) break;
        int32_t v = 0;
        for (int w = 0; w < nw; w++) v += part[w * FM * 256 + e];
        const int l = e & 63, rr = (e >> 6) & 3, i = e >> 8;
        const int mm = m0 + 16 * i + 4 * (l >> 4) + rr, nn = n0 + (l & 15);
        if (mm >= M || nn >= a.N) continue;
        const float p = (float)v * ews[j];
        float o = fmaf(p, sa[mm - m0], eb[j]);
        switch (a.act) {
        case 1: o = act_relu(o); break;
        case 2: o = act_gelu_tanh(o); break;
        case 3: o = act_gelu_erf(o); break;
        default: break;
        }
        a.out[(size_t)mm * a.ldo + nn] = a.accumulate ? eold[j] + o : o;
    }
}

// ------------------------------------------------------------- split K --

// out = epilogue(sum over the S chunk slices of the int32 partial products):
// the sums are exact, and the epilogue is epi_value, the expression every
// other kernel applies, so the outputs equal the unsplit GEMM's bit for bit.
// VEC: 4 consecutive outputs per thread (N, ldo multiples of 4, out aligned).
template <bool VEC>
__global__ __launch_bounds__(256) void gemm_i8_split_reduce(GemmArgs a, int S) {
    const int64_t MN = (int64_t)a.M * a.N;
    const int64_t step = (int64_t)gridDim.x * blockDim.x * (VEC ? 4 : 1);
    for (int64_t e = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * (VEC ? 4 : 1); e < MN; e += step) {
        const int m = (int)(e / a.N), n = (int)(e % a.N);
        if (VEC) {
            v4i acc = *reinterpret_cast<const v4i*>(a.split_ws + e);
            for (int z = 1; z < S; z++) acc += *reinterpret_cast<const v4i*>(a.split_ws + z * MN + e);
            float* o = a.out + (size_t)m * a.ldo + n;
            v4f v = {epi_value(a, m, n, acc.x), epi_value(a, m, n + 1, acc.y), epi_value(a, m, n + 2, acc.z),
                     epi_value(a, m, n + 3, acc.w)};
            if (a.accumulate) v = *reinterpret_cast<const v4f*>(o) + v;
            *reinterpret_cast<v4f*>(o) = v;
        } else {
            int32_t acc = a.split_ws[e];
            for (int z = 1; z < S; z++) acc += a.split_ws[z * MN + e];
            float* o = a.out + (size_t)m * a.ldo + n;
            const float v = epi_value(a, m, n, acc);
            *o = a.accumulate ? *o + v : v;
        }
    }
}

// --------------------------------------------------------------- generic --

__global__ __launch_bounds__(256) void gemm_i8_generic(GemmArgs a) {
    constexpr int BM = 64, BN = 64, BK = 64, SA = BK + 16, TM = 32, TN = 32;
    __shared__ __attribute__((aligned(16))) int8_t smem[(BM + BN) * SA];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    int tm, tn;
    tile_coords(blockIdx.x, (a.M + BM - 1) / BM, (a.N + BN - 1) / BN, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int K = a.K;
    // one A chunk and one B chunk per thread per slab
    const int r = tid >> 2, kc = (tid & 3) * 16;
    const bool aok = m0 + r < a.M, bok = n0 + r < a.N;
    const int8_t* arow = a.A + (size_t)(aok ? m0 + r : 0) * a.lda;
    const int8_t* brow = a.B + (size_t)(bok ? n0 + r : 0) * a.ldb;

    v4i acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = v4i{0, 0, 0, 0};

    for (int k0 = 0; k0 < K; k0 += BK) {
        const v4i va = aok ? load_chunk<false>(arow, k0 + kc, K) : v4i{0, 0, 0, 0};
        const v4i vb = bok ? load_chunk<false>(brow, k0 + kc, K) : v4i{0, 0, 0, 0};
        __syncthreads();
        *reinterpret_cast<v4i*>(smem + r * SA + kc) = va;
        *reinterpret_cast<v4i*>(smem + BM * SA + r * SA + kc) = vb;
        __syncthreads();
        v4i af[2], bf[2];
#pragma unroll
        for (int i = 0; i < 2; i++)
            af[i] = *reinterpret_cast<const v4i*>(smem + (wm * TM + i * 16 + (lane & 15)) * SA + (lane >> 4) * 16);
#pragma unroll
        for (int j = 0; j < 2; j++)
            bf[j] = *reinterpret_cast<const v4i*>(smem + BM * SA + (wn * TN + j * 16 + (lane & 15)) * SA +
                                                  (lane >> 4) * 16);
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) acc[i][j] = mfma_i8(af[i], bf[j], acc[i][j]);
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + wn * TN + j * 16 + (lane & 15);
            if (n >= a.N) continue;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int m = m0 + wm * TM + i * 16 + 4 * (lane >> 4) + q;
                if (m < a.M) store_out(a, m, n, acc[i][j][q]);
            }
        }
}

// ---------------------------------------------------------------- launch --

constexpr int kCUs = 256;

template <int BM, int BN, int BK>
void run_tiled(const GemmArgs& a, hipStream_t st, int splits = 1) {
    using C = TileCfg<BM, BN, BK>;
    static const bool attr = [] {
        // above 64 KiB a kernel must opt in to the larger LDS allocation
        if (C::LDS > 65536)
            VLA_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_i8_tiled<BM, BN, BK>),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS));
        return true;
    }();
    (void)attr;
    const int blocks = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    gemm_i8_tiled<BM, BN, BK><<<dim3(blocks, splits), 256, C::LDS, st>>>(a);
    VLA_LAUNCH_CHECK();
}

template <int BM, int BN, int BK, int S, int WM = 2, int WN = 2, bool PF = false, bool CONV = false,
          bool IMPL = false>
void run_lds(const GemmArgs& a, hipStream_t st) {
    using C = LdsCfg<BM, BN, BK, S, WM, WN>;
    static const bool attr = [] {
        if (C::LDS > 65536)
            VLA_HIP_CHECK(hipFuncSetAttribute(
                reinterpret_cast<const void*>(&gemm_i8_lds<BM, BN, BK, S, WM, WN, PF, CONV, IMPL>),
                hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS));
        return true;
    }();
    (void)attr;
    const int blocks = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    gemm_i8_lds<BM, BN, BK, S, WM, WN, PF, CONV, IMPL><<<blocks, C::NT, C::LDS, st>>>(a);
    VLA_LAUNCH_CHECK();
}

// Row groups of the skinny kernel: each block owns 16 columns and FM of the
// M / 16 row fragments, so a narrow output (N / 16 well under the CU count)
// still spreads over the chip and each block reads only its rows of A.
// VLA_HIP_SKINNY_R=<groups> forces a count (A/B runs; values unchanged).
// Default: the fewest groups that give every CU a block. Measured on MI355X
// (graph replays, forced counts 1/2/3/4/8): 100x2560x960 9.94 -> 5.29 us
// (4 groups), 50x720x960 4.09 -> 3.06 (4), 50x2048x720 6.12 -> 4.33 (4),
// 100x512x3200 5.20 -> 4.82 (2); at N = 4096 (256 column blocks) one group
// is fastest over K = 4096 (50 rows: 9.85 us, 12.19 with two), since more
// only re-read the weights, but two win over a short K (50x720x4096 4.63 ->
// 4.43 us).
int skinny_row_groups(int M, int N, int K, int S, int fn = 1) {
    const int nfrag = (M + 15) / 16;
    const char* env = std::getenv("VLA_HIP_SKINNY_R");
    const long blocks = (long)((N + 16 * fn - 1) / (16 * fn)) * (S > 1 ? S : 1);
    int g = (int)((kCUs + blocks - 1) / blocks);
    if (K <= 1024 && g < 2) g = 2;
    if (env && *env) g = std::atoi(env);
    if (fn > 1 && g < (nfrag + 3) / 4) g = (nfrag + 3) / 4;  // two column groups hold at most 4 fragments
    g = g < 1 ? 1 : g > nfrag ? nfrag : g;
    const int fm = (nfrag + g - 1) / g;
    return (nfrag + fm - 1) / fm;
}

// Column groups per skinny block (16 x FN columns): two where more than 64
// rows meet a long K and a wide output, VLA_HIP_SKINNY_FN=1|2 forces a count
// (A/B runs). Graph replays on MI355X, one -> two: 100x4096x4096 13.75 ->
// 12.33 us (each block reads half as much of A per column; with two row
// groups a CU still moves 393 instead of 524 KB), but 50x4096x4096 9.96 ->
// 10.06, 100x768x3072 5.52 -> 6.92, 100x512x3200 4.81 -> 6.44, 100x2560x960
// 5.35 -> 6.36, SmolVLA chunk 6.86 -> 7.02 ms.
int skinny_col_groups(int M, int N, int K) {
    const char* env = std::getenv("VLA_HIP_SKINNY_FN");
    if (env && *env) return std::atoi(env) == 2 && M > 16 ? 2 : 1;
    return M > 64 && K >= 2048 && N >= 4096 ? 2 : 1;
}

// Two column groups per block: at most 4 fragments and 8 waves (the partial
// tiles' LDS), no rotating epilogue.
template <int WAVES>
void run_skinny_fn2(const GemmArgs& a, hipStream_t st, int splits, int groups) {
    const int fm = ((a.M + 15) / 16 + groups - 1) / groups;
    const dim3 nb((a.N + 31) / 32, splits, groups);
    constexpr int W = WAVES < 8 ? WAVES : 8;
    switch (fm) {
    case 1: gemm_i8_skinny<1, W, false, 2><<<nb, W * 64, 0, st>>>(a); break;
    case 2: gemm_i8_skinny<2, W, false, 2><<<nb, W * 64, 0, st>>>(a); break;
    case 3: gemm_i8_skinny<3, W, false, 2><<<nb, W * 64, 0, st>>>(a); break;
    default: gemm_i8_skinny<4, W, false, 2><<<nb, W * 64, 0, st>>>(a); break;
    }
    VLA_LAUNCH_CHECK();
}

template <int WAVES, bool ROPE = false>
void run_skinny(const GemmArgs& a, hipStream_t st, int splits = 1, int groups = 1, int fn = 1) {
    if constexpr (!ROPE) {
        if (fn == 2) {
            run_skinny_fn2<WAVES>(a, st, splits, groups);
            return;
        }
    }
    const int fm = ((a.M + 15) / 16 + groups - 1) / groups;
    const dim3 nb((a.N + 15) / 16, splits, groups);
    constexpr int W8 = WAVES < 8 ? WAVES : 8;  // FM > 4 keeps the partial tiles within 64 KiB
    switch (fm) {
    case 1: gemm_i8_skinny<1, WAVES, ROPE><<<nb, WAVES * 64, 0, st>>>(a); break;
    case 2: gemm_i8_skinny<2, WAVES, ROPE><<<nb, WAVES * 64, 0, st>>>(a); break;
    case 3: gemm_i8_skinny<3, WAVES, ROPE><<<nb, WAVES * 64, 0, st>>>(a); break;
    case 4: gemm_i8_skinny<4, WAVES, ROPE><<<nb, WAVES * 64, 0, st>>>(a); break;
    case 5: gemm_i8_skinny<5, W8, ROPE><<<nb, W8 * 64, 0, st>>>(a); break;
    case 6: gemm_i8_skinny<6, W8, ROPE><<<nb, W8 * 64, 0, st>>>(a); break;
    case 7: gemm_i8_skinny<7, W8, ROPE><<<nb, W8 * 64, 0, st>>>(a); break;
    default: gemm_i8_skinny<8, W8, ROPE><<<nb, W8 * 64, 0, st>>>(a); break;
    }
    VLA_LAUNCH_CHECK();
}

template <int MV>
void run_gemv_m(const GemmArgs& a, hipStream_t st) {
    const int nch = (a.K + 15) / 16;
    if (nch >= 48) gemm_i8_gemv<MV, 64><<<(a.N + 3) / 4, 256, 0, st>>>(a);
    else if (nch >= 24) gemm_i8_gemv<MV, 32><<<(a.N + 7) / 8, 256, 0, st>>>(a);
    else gemm_i8_gemv<MV, 16><<<(a.N + 15) / 16, 256, 0, st>>>(a);
    VLA_LAUNCH_CHECK();
}

void run_gemv(const GemmArgs& a, hipStream_t st) {
    if (a.M == 1) run_gemv_m<1>(a, st);
    else run_gemv_m<2>(a, st);
}

// One or two rows over K >= 2048 take gemm_i8_gemv (VLA_HIP_GEMV=0 turns it
// off). Graph replays on MI355X, skinny -> gemv: 1x4096x4096 6.44 -> 5.48 us,
// 2x4096x4096 6.47 -> 6.05, 1x2560x960 4.84 -> 3.45, 1x2048x720 4.20 -> 3.10;
// but 4x4096x4096 6.47 -> 7.66 and, over K <= 1024, 1x512x3200 3.18 -> 3.33
// (the skinny kernel's short rows are already one load round trip).
bool use_gemv(int M, int K) {
    static const bool on = [] {
        const char* e = std::getenv("VLA_HIP_GEMV");
        return !(e && e[0] == '0');
    }();
    return on && M <= 2 && K >= 2048;
}

template <int OP, int NV, int FM>
void run_rowop(const RowQArgs& r, const GemmArgs& a, hipStream_t st) {
    static const bool attr = [] {
        VLA_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_i8_rowop<OP, NV, FM>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, kRowopMaxLds));
        return true;
    }();
    (void)attr;
    const int lds = rowop_lds_main(FM, a.K) + 16 * FM * 4;
    const dim3 grid((a.N + 15) / 16, (a.M + 16 * FM - 1) / (16 * FM));
    gemm_i8_rowop<OP, NV, FM><<<grid, 1024, lds, st>>>(r, a);
    VLA_LAUNCH_CHECK();
}

// Rows per block of the fused row-op GEMM (16 x FM, FM in 1, 2, 4, 8): as the
// skinny kernel's row groups, the fewest groups that give every CU a block
// (each block then applies the row op to its own rows only), or
// VLA_HIP_ROWOP_R=<groups>.
int rowop_group_fm(int M, int N) {
    const char* env = std::getenv("VLA_HIP_ROWOP_R");
    const int nb = (N + 15) / 16;
    int g = (kCUs + nb - 1) / nb;
    if (env && *env) g = std::atoi(env);
    g = g < 1 ? 1 : g;
    return rowop_fm((M + g - 1) / g);
}

template <int OP, int NV>
void run_rowop_fm(const RowQArgs& r, const GemmArgs& a, hipStream_t st) {
    switch (rowop_group_fm(a.M, a.N)) {
    case 1: run_rowop<OP, NV, 1>(r, a, st); break;
    case 2: run_rowop<OP, NV, 2>(r, a, st); break;
    case 4: run_rowop<OP, NV, 4>(r, a, st); break;
    default:
        if constexpr (NV <= 4) run_rowop<OP, NV, 8>(r, a, st);
        else throw ArgError("gemm_i8_rowop: 128 rows need K <= 1024");
        break;
    }
}

template <int OP>
void run_rowop_nv(const RowQArgs& r, const GemmArgs& a, hipStream_t st) {
    const int nv = (a.K + 255) / 256;
    if (nv <= 1) run_rowop_fm<OP, 1>(r, a, st);
    else if (nv <= 2) run_rowop_fm<OP, 2>(r, a, st);
    else if (nv <= 4) run_rowop_fm<OP, 4>(r, a, st);
    else run_rowop_fm<OP, 8>(r, a, st);
}

// Tile of the aligned kernel: the largest that still gives every CU a tile,
// or VLA_HIP_GEMM_TILE=<BM>x<BN>x<BK> to force one (A/B runs; the values do
// not change, only the schedule).
// stages == 0: the register-staged gemm_i8_tiled; > 0: gemm_i8_lds with that
// many LDS stages (named "<BM>x<BN>x<BK>s<S>").
struct Tile {
    int bm, bn, bk, stages, waves = 4;
    bool pf = false;  // fragment-pipelined main loop (gemm_i8_lds PF)
};
const Tile kTiles[] = {{128, 128, 64, 0},       {64, 128, 64, 0},         {64, 64, 64, 0},
                       {64, 64, 128, 0},        {64, 128, 128, 0},
                       {128, 128, 64, 4},       {64, 128, 64, 4},         {256, 128, 128, 3, 8},
                       {256, 256, 128, 2, 8},   {256, 128, 128, 3, 8, true}, {256, 256, 128, 2, 8, true},
                       {128, 128, 128, 2},      {64, 64, 128, 3},         {64, 64, 128, 4},
                       {32, 64, 128, 3},        {32, 64, 128, 4}};

Tile pick_tile(int M, int N, int K) {
    const char* env = std::getenv("VLA_HIP_GEMM_TILE");
    if (env && *env) {
        for (const Tile& t : kTiles) {
            char name[32];
            if (t.stages && (t.waves != 4 || t.pf))
                std::snprintf(name, sizeof name, "%dx%dx%ds%dw%d%s", t.bm, t.bn, t.bk, t.stages, t.waves,
                              t.pf ? "p" : "");
            else if (t.stages)
                std::snprintf(name, sizeof name, "%dx%dx%ds%d", t.bm, t.bn, t.bk, t.stages);
            else
                std::snprintf(name, sizeof name, "%dx%dx%d", t.bm, t.bn, t.bk);
            if (std::strcmp(name, env) == 0) return t;
        }
    }
    // Measured on MI355X over the BASELINE sweep (bench.py, forced tiles):
    // short K (<= 1024) is dominated by the fp32 output write and wants many
    // small register-staged tiles in flight: 64 x 128 only from two such tiles
    // per CU (Octo's 658 x 3072 x 768 MLP runs faster as 528 64 x 64 tiles than
    // as 264 64 x 128 ones: 1.227 -> 1.183 ms per forward). Long K wants the LDS-DMA pipeline
    // with the largest tile that still fills the chip: 256 x 256 with 8 waves
    // when there are two tiles per CU, else 256 x 128 with 8 waves when every
    // CU gets a tile, else smaller tiles; the fragment-pipelined main loop
    // (PF) is 5-8% faster than the plain one on both large tiles. A 4-wave
    // 256 x 256 form needs more than 256 VGPRs for its fragments and
    // accumulators, and spills.
    auto tiles = [&](int bm, int bn) { return (long)((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    // 64 x 64 tiles walk K in 128-byte slabs once K has two of them: half the
    // barriers and twice the MFMA work per slab (ACT 0.409 -> 0.402 ms, Octo
    // 1.159 -> 1.141 ms per forward)
    const Tile small{64, 64, K >= 256 ? 128 : 64, 0};
    // The policy layers' GEMMs (a few hundred to ~1000 rows, tiles < 2 per CU)
    // take the LDS-DMA 64 x 64 tile with 128-byte slabs: every slab of a short
    // K is in flight at once (3 stages, 48 KiB: three blocks per CU), 4 stages
    // over long K. Interleaved repeats on MI355X, register-staged / split-K
    // tile -> this: 1024x768x2304 8.70 -> 7.51 us, 658x768x3072 8.62 -> 7.36,
    // 302x512x3200 5.67 -> 4.89, 177x960x2560 7.25 -> 6.09, 1024x3072x768
    // 16.98 -> 11.23, 2048x2560x960 15.59 -> 11.86, 512x4096x4096 23.97 ->
    // 20.12, 512x2560x960 13.80 -> 9.90; bit-identical sums. Very long K over
    // at most 64 such tiles (302x3200x512 10.38 split vs 11.27, 200x4096x1024
    // 12.96 vs 13.61) stays on the split-K register tile.
    // Where 64 x 64 tiles leave CUs idle and 32 x 64 ones number at most 1.5
    // per CU (Octo's 658/690 x 768 outputs: 132 -> 252/264 blocks, SigLIP's
    // 1024 x 768: 192 -> 384), the 32 x 64 tile with 4 stages: a block then
    // pulls (32 + 64) instead of (64 + 64) bytes per byte of K, and the
    // per-CU L2 -> LDS fill is what these layers wait on. Forced tiles, graph
    // replays: 690x3072x768 10.94 -> 10.59 us (3 stages 11.02), 690x768x768
    // 5.15 -> 4.86 (4.98), 1024x768x768 5.14 -> 4.97 (5.12), 1024x3072x768
    // 10.93 -> 10.60 (10.97). VLA_HIP_GEMM_T32=0 keeps the 64 x 64 tile (A/B
    // runs; sums unchanged).
    const char* t32 = std::getenv("VLA_HIP_GEMM_T32");
    const bool use32 =
        tiles(64, 64) < kCUs && tiles(32, 64) <= kCUs + kCUs / 2 && !(t32 && std::atoi(t32) == 0);
    const Tile lds = use32 ? Tile{32, 64, 128, 4} : Tile{64, 64, 128, K <= 1024 ? 3 : 4};
    // Large outputs over short K (M, N >= 1024, 512 <= K <= 1024, at least
    // one 128 x 128 tile per CU): the LDS-DMA 128 x 128 tile with 128-byte
    // slabs, two stages (64 KiB, two blocks per CU) and non-temporal stores;
    // interleaved repeats on MI355X: 8192 x 768 x 3072 46.6 -> 37.0 us,
    // 8192 x 960 x 2560 47.5 -> 38.3, 2048 x 768 x 3072 13.2 -> 11.5,
    // 2048 x 512 x 3200 12.0 -> 9.8. With fewer tiles than CUs (SigLIP's
    // 1024-row layers), at 658 rows and at 1000^3 the register-staged tiles
    // stay ahead.
    if (K <= 1024 && K >= 512 && M >= 1024 && N >= 1024 && tiles(128, 128) >= kCUs) return {128, 128, 128, 2};
    if (K <= 1024) return tiles(64, 128) >= 2 * kCUs ? Tile{64, 128, 64, 0} : K >= 256 ? lds : small;
    if (tiles(256, 256) >= 2 * kCUs) return {256, 256, 128, 2, 8, true};
    if (tiles(256, 128) >= kCUs) return {256, 128, 128, 3, 8, true};
    if (tiles(128, 128) >= kCUs) return {128, 128, 64, 4};
    if (tiles(64, 64) <= 64 && K >= 3072) return small;  // split over K (split_plan)
    return lds;
}

// Split-K plan: for M > 128 on the register-staged tiles with K >= 1024 and
// fewer tiles than CUs, S chunks of K (multiples of 128 bytes, each >= 512)
// so that S x tiles reaches about two blocks per CU, S <= 8. S x tiles <= 2 x
// CUs bounds the workspace: S x M x N <= 512 x 64 x 64 int32s (8 MiB).
// Measured on MI355X: splitting the LDS-DMA tiles when they number one per
// CU made 512 x 4096 x 4096 and 2048 x 960 x 2560 slower (23.7 -> 31.5 and
// 16.1 -> 27.4 us: the partial sums' round trip costs more than the idle
// half of each CU), so those keep one launch.
struct SplitPlan {
    int S = 1, kchunk = 0;
};
// The skinny kernel (M <= 128) runs one block per 16 columns; with fewer
// than half a block per CU and K >= 8192 it splits K into S <= 8 chunks of
// >= 2048 bytes (multiples of 128) so that S x blocks is about one per CU.
// Below K = 8192 the reduce launch costs more than the idle CUs: graph
// replays on MI355X (panel rows, rotating weights), unsplit -> split:
// 8x1024x5120 6.15 -> 7.35 us, 4x2048x5120 6.30 -> 7.64, 4x1024x4096 5.36
// -> 6.67; above it the split wins: 4x1024x20480 16.0 -> 9.80, 8x512x10240
// 9.37 -> 7.80, 4x2048x10240 9.75 -> 9.36 (Diffusion Policy's UNet shapes).
SplitPlan skinny_split_plan(int N, int K) {
    SplitPlan p;
    const int nb = (N + 15) / 16;
    if (K < 8192 || 2 * nb > kCUs) return p;
    int S = kCUs / nb;
    S = S < 8 ? S : 8;
    S = S < K / 2048 ? S : K / 2048;
    if (S < 2) return p;
    p.kchunk = ((K + S - 1) / S + 127) / 128 * 128;
    p.S = (K + p.kchunk - 1) / p.kchunk;
    if (p.S < 2) p = SplitPlan{};
    return p;
}

// 129..320 row-major rows over a narrow output (N <= 2048: at most 128
// column blocks, where the tiles leave most CUs idle) take the skinny kernel
// in row groups of at most 8 fragments, unsplit. Graph replays on MI355X,
// tiles -> skinny: 177x960x960 5.87 -> 4.30 us, 177x960x320 5.65 -> 3.00,
// 177x2560x960 9.82 -> 7.53, 256x960x960 5.81 -> 4.79, 200x4096x1024 13.5 ->
// 12.0; wide outputs stay on the tiles (177x960x5120 6.63 -> 12.76). ACT's
// 302-row encoder (40 tiles of 64 x 64 per 512-wide projection, its w2 split
// over K with a reduce pass) 0.343 -> 0.325 ms per forward with the bound at
// 320; Octo's 658 rows lose on it (1.06 -> 1.21 ms with the bound at 704).
// VLA_HIP_SKINNY_MAXM=<rows> moves the route's upper bound (128 turns it
// off), and a tile forced with VLA_HIP_GEMM_TILE bypasses it (both read per
// call, like the other knobs).
bool skinny_mid_rows(int M, int N, bool panel) {
    if (M <= 128 || N > 2048 || panel) return false;
    const char* tile = std::getenv("VLA_HIP_GEMM_TILE");
    if (tile && *tile) return false;
    const char* e = std::getenv("VLA_HIP_SKINNY_MAXM");
    const int maxm = e && std::atoi(e) >= 128 ? std::atoi(e) : 320;
    return M <= maxm;
}

SplitPlan split_plan(int M, int N, int K) {
    SplitPlan p;
    if (M <= kPanelMaxRows) return skinny_split_plan(N, K);
    if (skinny_mid_rows(M, N, false)) return p;
    if (K < 1024) return p;
    const Tile t = pick_tile(M, N, K);
    if (t.stages != 0) return p;
    const long tiles = (long)((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
    if (tiles >= kCUs) return p;
    int S = (int)(2 * kCUs / tiles);
    S = S < 8 ? S : 8;
    S = S < K / 512 ? S : K / 512;
    if (S < 2) return p;
    p.kchunk = ((K + S - 1) / S + 127) / 128 * 128;
    p.S = (K + p.kchunk - 1) / p.kchunk;
    if (p.S < 2) p = SplitPlan{};
    return p;
}

void dispatch_tile(const Tile& t, const GemmArgs& a, hipStream_t st) {
    if (t.stages && t.waves == 8) {
        if (t.bn == 256 && t.pf) run_lds<256, 256, 128, 2, 2, 4, true>(a, st);
        else if (t.bn == 256) run_lds<256, 256, 128, 2, 2, 4>(a, st);
        else if (t.pf) run_lds<256, 128, 128, 3, 4, 2, true>(a, st);
        else run_lds<256, 128, 128, 3, 4, 2>(a, st);
        return;
    }
    if (t.stages) {
        if (t.bm == 32) {
            if (t.stages == 3) run_lds<32, 64, 128, 3>(a, st);
            else run_lds<32, 64, 128, 4>(a, st);
        } else if (t.bm == 64 && t.bn == 64) {
            if (t.stages == 3) run_lds<64, 64, 128, 3>(a, st);
            else run_lds<64, 64, 128, 4>(a, st);
        } else if (t.bm == 128 && t.bk == 128) run_lds<128, 128, 128, 2>(a, st);
        else if (t.bm == 128) run_lds<128, 128, 64, 4>(a, st);
        else run_lds<64, 128, 64, 4>(a, st);
        return;
    }
    if (t.bm == 128) run_tiled<128, 128, 64>(a, st);
    else if (t.bn == 128 && t.bk == 128) run_tiled<64, 128, 128>(a, st);
    else if (t.bn == 128) run_tiled<64, 128, 64>(a, st);
    else if (t.bk == 128) run_tiled<64, 64, 128>(a, st);
    else run_tiled<64, 64, 64>(a, st);
}

}  // namespace

void launch_gemm_i8(const GemmArgs& a, hipStream_t st) {
    VLA_REQUIRE(a.M >= 0 && a.N > 0 && a.K > 0, "gemm_i8: need M >= 0, N > 0, K > 0");
    VLA_REQUIRE(a.K <= kMaxI8K, "gemm_i8: K exceeds the int8 accumulator bound INT_MAX/(255*127)");
    VLA_REQUIRE((a.a_panel || (a.lda >= kpad4(a.K) && a.lda % 4 == 0)) && a.ldb >= kpad4(a.K) && a.ldb % 4 == 0,
                "gemm_i8: int8 row strides must be multiples of 4 and >= i8_kpad(K)");
    VLA_REQUIRE(aligned(a.A, 4) && aligned(a.B, 4), "gemm_i8: int8 operands must be 4-byte aligned");
    VLA_REQUIRE(a.acc32 || (a.out && a.wscale && a.ascale && a.ldo >= a.N),
                "gemm_i8: fp32 output needs out, wscale, ascale and ldo >= N");
    VLA_REQUIRE(a.act >= 0 && a.act <= 3, "gemm_i8: unknown activation");
    if (a.M == 0) return;

    const bool al = (a.a_panel || a.lda % 16 == 0) && a.ldb % 16 == 0 && aligned(a.A, 16) &&
                    aligned(a.B, 16) && (a.acc32 ? aligned(a.acc32, 16) : aligned(a.out, 16));
    VLA_REQUIRE(!a.a_panel || (a.M <= kPanelMaxRows && al),
                "gemm_i8: panel-layout activations need M <= 128 and 16-byte aligned operands");
    VLA_REQUIRE(!a.rope_cs || (al && a.M <= 128 && !a.acc32 && a.act == 0 && !a.accumulate && a.rope_hd > 0 &&
                               a.rope_hd % 16 == 0 && a.rope_cols > 0 && a.rope_cols % a.rope_hd == 0 &&
                               a.rope_cols <= a.N),
                "gemm_i8: the rotating epilogue needs M <= 128, aligned operands, fp32 output without "
                "activation or accumulation, and whole heads of a multiple of 16 columns");
    if (!al) {
        const int blocks = ((a.M + 63) / 64) * ((a.N + 63) / 64);
        gemm_i8_generic<<<blocks, 256, 0, st>>>(a);
        VLA_LAUNCH_CHECK();
        return;
    }
    if (a.rope_cs) {
        const int steps = (a.K + 63) / 64, g = skinny_row_groups(a.M, a.N, a.K, 1);
        if (steps >= 32) run_skinny<16, true>(a, st, 1, g);
        else if (steps >= 8) run_skinny<8, true>(a, st, 1, g);
        else run_skinny<4, true>(a, st, 1, g);
        return;
    }
    if (use_gemv(a.M, a.K)) {
        run_gemv(a, st);
        return;
    }
    if (skinny_mid_rows(a.M, a.N, a.a_panel)) {
        const int nfrag = (a.M + 15) / 16, steps = (a.K + 63) / 64;
        int g = skinny_row_groups(a.M, a.N, a.K, 1);
        g = g < (nfrag + 7) / 8 ? (nfrag + 7) / 8 : g;
        if (steps >= 32) run_skinny<16>(a, st, 1, g);
        else if (steps >= 8) run_skinny<8>(a, st, 1, g);
        else run_skinny<4>(a, st, 1, g);
        return;
    }
    if (a.M <= 128) {
        SplitPlan p;
        if (a.split_ws && !a.acc32) {
            p = split_plan(a.M, a.N, a.K);
            if (p.S > 1 && !(a.split_bytes >= (size_t)p.S * a.M * a.N * 4 && aligned(a.split_ws, 16))) p = SplitPlan{};
        }
        GemmArgs s = a;
        s.kchunk = p.kchunk;
        const int fn = skinny_col_groups(a.M, a.N, a.K);
        const int steps = ((p.S > 1 ? p.kchunk : a.K) + 63) / 64, g = skinny_row_groups(a.M, a.N, a.K, p.S, fn);
        if (steps >= 32) run_skinny<16>(s, st, p.S, g, fn);
        else if (steps >= 8) run_skinny<8>(s, st, p.S, g, fn);
        else run_skinny<4>(s, st, p.S, g, fn);
        if (p.S > 1) {
            const bool vec = a.N % 4 == 0 && a.ldo % 4 == 0 && aligned(a.out, 16);
            const int64_t work = (int64_t)a.M * a.N / (vec ? 4 : 1);
            const int blocks = (int)((work + 255) / 256 < 4096 ? (work + 255) / 256 : 4096);
            if (vec) gemm_i8_split_reduce<true><<<blocks, 256, 0, st>>>(s, p.S);
            else gemm_i8_split_reduce<false><<<blocks, 256, 0, st>>>(s, p.S);
            VLA_LAUNCH_CHECK();
        }
        return;
    }
    const Tile t = pick_tile(a.M, a.N, a.K);
    if (a.split_ws && !a.acc32) {
        const SplitPlan p = split_plan(a.M, a.N, a.K);
        if (p.S > 1 && a.split_bytes >= (size_t)p.S * a.M * a.N * 4 && aligned(a.split_ws, 16)) {
            GemmArgs s = a;
            s.kchunk = p.kchunk;
            if (t.bm == 128) run_tiled<128, 128, 64>(s, st, p.S);
            else if (t.bn == 128) run_tiled<64, 128, 64>(s, st, p.S);
            else if (t.bk == 128) run_tiled<64, 64, 128>(s, st, p.S);
            else run_tiled<64, 64, 64>(s, st, p.S);
            const bool vec = a.N % 4 == 0 && a.ldo % 4 == 0 && aligned(a.out, 16);
            const int64_t work = (int64_t)a.M * a.N / (vec ? 4 : 1);
            const int blocks = (int)((work + 255) / 256 < 4096 ? (work + 255) / 256 : 4096);
            if (vec) gemm_i8_split_reduce<true><<<blocks, 256, 0, st>>>(s, p.S);
            else gemm_i8_split_reduce<false><<<blocks, 256, 0, st>>>(s, p.S);
            VLA_LAUNCH_CHECK();
            return;
        }
    }
    dispatch_tile(t, a, st);
}

// The kernel choice of launch_gemm_i8 above for the shapes whose kernels
// carry the convolution epilogue; anything else returns 0 unlaunched.
int launch_gemm_i8_conv(const GemmArgs& a, hipStream_t st) {
    if (!a.omax || a.acc32 || a.accumulate || a.a_panel || a.rope_cs || a.M <= 0 || a.N <= 0 || a.K <= 0 ||
        a.K > kMaxI8K || !a.out || !a.wscale || !a.ascale || a.ldo < a.N || a.ldo % 4 != 0)
        return 0;
    if (a.resid ? a.act != 0 : a.act != 1) return 0;
    if (a.lda % 16 != 0 || a.ldb % 16 != 0 || a.lda < kpad4(a.K) || a.ldb < kpad4(a.K) || !aligned(a.A, 16) ||
        !aligned(a.B, 16) || !aligned(a.out, 16) || (a.resid && !aligned(a.resid, 16)) || use_gemv(a.M, a.K))
        return 0;
    if (skinny_mid_rows(a.M, a.N, false)) {
        const int nfrag = (a.M + 15) / 16, steps = (a.K + 63) / 64;
        int g = skinny_row_groups(a.M, a.N, a.K, 1);
        g = g < (nfrag + 7) / 8 ? (nfrag + 7) / 8 : g;
        const int parts = (a.N + 15) / 16 * g;  // one per block
        if (parts > kConvPartsFused) return 0;
        if (steps >= 32) run_skinny<16>(a, st, 1, g);
        else if (steps >= 8) run_skinny<8>(a, st, 1, g);
        else run_skinny<4>(a, st, 1, g);
        return parts;
    }
    if (a.M <= 128) return 0;
    if (a.split_ws) {
        const SplitPlan p = split_plan(a.M, a.N, a.K);
        if (p.S > 1 && a.split_bytes >= (size_t)p.S * a.M * a.N * 4 && aligned(a.split_ws, 16)) return 0;
    }
    const Tile t = pick_tile(a.M, a.N, a.K);
    if (!(t.bm == 32 && t.stages == 4 && t.waves == 4 && !t.pf)) return 0;
    const int64_t parts = (int64_t)((a.M + 31) / 32) * ((a.N + 63) / 64);  // one per block
    if (parts > kConvPartsFused) return 0;
    run_lds<32, 64, 128, 4, 2, 2, false, true>(a, st);
    return (int)parts;
}

int launch_gemm_i8_conv_implicit(const GemmArgs& a, hipStream_t st) {
    VLA_REQUIRE(a.cv_c > 0 && a.cv_c % 64 == 0 && a.cv_k > 0 && a.cv_s > 0 && a.cv_p >= 0 && a.cv_wo > 0 &&
                    a.cv_h > 0 && a.cv_w > 0 && a.K == a.cv_k * a.cv_k * a.cv_c && a.K <= kMaxI8K && a.M > 0 &&
                    a.N > 0,
                "gemm_i8 implicit conv: need 64-channel multiples and K = k * k * Cin");
    VLA_REQUIRE(aligned(a.A, 16) && aligned(a.B, 16) && a.ldb % 16 == 0 && a.ldb >= a.K && aligned(a.out, 16) &&
                    a.ldo % 4 == 0 && a.ldo >= a.N && a.wscale && a.ascale && !a.acc32 && !a.accumulate &&
                    !a.a_panel && !a.rope_cs,
                "gemm_i8 implicit conv: 16-byte aligned operands, fp32 output, no accumulation");
    const int64_t blocks = (int64_t)((a.M + 31) / 32) * ((a.N + 63) / 64);
    if (a.omax) {
        VLA_REQUIRE((a.resid ? a.act == 0 : a.act == 1) && blocks <= kConvPartsFused &&
                        (!a.resid || aligned(a.resid, 16)),
                    "gemm_i8 implicit conv: bad fused epilogue");
        run_lds<32, 64, 128, 4, 2, 2, false, true, true>(a, st);
        return (int)blocks;
    }
    VLA_REQUIRE(!a.resid, "gemm_i8 implicit conv: a residual needs omax");
    run_lds<32, 64, 128, 4, 2, 2, false, false, true>(a, st);
    return 0;
}

namespace {

template <int WAVES>
void run_skinny_implicit(const GemmArgs& a, hipStream_t st, int groups) {
    const int fm = ((a.M + 15) / 16 + groups - 1) / groups;
    const dim3 nb((a.N + 15) / 16, 1, groups);
    constexpr int W8 = WAVES < 8 ? WAVES : 8;
    switch (fm) {
    case 1: gemm_i8_skinny<1, WAVES, false, 1, true><<<nb, WAVES * 64, 0, st>>>(a); break;
    case 2: gemm_i8_skinny<2, WAVES, false, 1, true><<<nb, WAVES * 64, 0, st>>>(a); break;
    case 3: gemm_i8_skinny<3, WAVES, false, 1, true><<<nb, WAVES * 64, 0, st>>>(a); break;
    case 4: gemm_i8_skinny<4, WAVES, false, 1, true><<<nb, WAVES * 64, 0, st>>>(a); break;
    case 5: gemm_i8_skinny<5, W8, false, 1, true><<<nb, W8 * 64, 0, st>>>(a); break;
    case 6: gemm_i8_skinny<6, W8, false, 1, true><<<nb, W8 * 64, 0, st>>>(a); break;
    case 7: gemm_i8_skinny<7, W8, false, 1, true><<<nb, W8 * 64, 0, st>>>(a); break;
    default: gemm_i8_skinny<8, W8, false, 1, true><<<nb, W8 * 64, 0, st>>>(a); break;
    }
    VLA_LAUNCH_CHECK();
}

}  // namespace

bool gemm_i8_conv_skinny_fits(int M, int N) {
    // VLA_HIP_CONV_SKINNY_MAXM (read per call): the most output pixels, default 320
    const char* e = std::getenv("VLA_HIP_CONV_SKINNY_MAXM");
    const int maxm = e && std::atoi(e) > 128 ? std::atoi(e) : 320;
    return M > 128 && M <= maxm && N <= 2048;
}

int launch_gemm_i8_conv_skinny_implicit(const GemmArgs& a, hipStream_t st) {
    VLA_REQUIRE(a.cv_c > 0 && a.cv_c % 64 == 0 && a.cv_k > 0 && a.cv_s > 0 && a.cv_p >= 0 && a.cv_wo > 0 &&
                    a.cv_h > 0 && a.cv_w > 0 && a.K == a.cv_k * a.cv_k * a.cv_c && a.K <= kMaxI8K && a.M > 128 &&
                    a.N <= 2048,
                "gemm_i8 skinny implicit conv: need 64-channel multiples, K = k * k * Cin, > 128 rows, N <= 2048");
    VLA_REQUIRE(aligned(a.A, 16) && aligned(a.B, 16) && a.ldb % 16 == 0 && a.ldb >= a.K && a.out && a.wscale &&
                    a.ascale && a.ldo >= a.N && !a.acc32 && !a.accumulate && !a.a_panel && !a.rope_cs,
                "gemm_i8 skinny implicit conv: 16-byte aligned operands, fp32 output, no accumulation");
    const int nfrag = (a.M + 15) / 16, steps = a.K / 64;
    int g = skinny_row_groups(a.M, a.N, a.K, 1);
    g = g < (nfrag + 7) / 8 ? (nfrag + 7) / 8 : g;
    const int parts = (a.N + 15) / 16 * g;
    VLA_REQUIRE(!a.omax || ((a.resid ? a.act == 0 : a.act == 1) && parts <= kConvPartsFused),
                "gemm_i8 skinny implicit conv: bad fused epilogue");
    VLA_REQUIRE(a.omax || !a.resid, "gemm_i8 skinny implicit conv: a residual needs omax");
    if (steps >= 32) run_skinny_implicit<16>(a, st, g);
    else if (steps >= 8) run_skinny_implicit<8>(a, st, g);
    else run_skinny_implicit<4>(a, st, g);
    return a.omax ? parts : 0;
}

namespace {

// Whether launch_gemm_i8 would run a through run_skinny in one unsplit launch
// with one column group per block (no rotating epilogue, no int32 output).
bool plain_skinny(const GemmArgs& a) {
    const bool al = (a.a_panel || a.lda % 16 == 0) && a.ldb % 16 == 0 && aligned(a.A, 16) && aligned(a.B, 16) &&
                    aligned(a.out, 16);
    if (!al || a.rope_cs || a.acc32 || a.M <= 0 || use_gemv(a.M, a.K)) return false;
    if (skinny_mid_rows(a.M, a.N, a.a_panel)) return true;
    if (a.M > 128) return false;
    if (a.split_ws && split_plan(a.M, a.N, a.K).S > 1) return false;
    return skinny_col_groups(a.M, a.N, a.K) == 1;
}

int skinny_waves(int K) {
    const int steps = (K + 63) / 64;
    return steps >= 32 ? 16 : steps >= 8 ? 8 : 4;
}

template <int WAVES>
void run_skinny_pair(const GemmArgs& a1, const GemmArgs& a2, int fm, int groups, hipStream_t st) {
    const int nb1 = (a1.N + 15) / 16;
    const dim3 nb(nb1 + (a2.N + 15) / 16, 1, groups);
    constexpr int W8 = WAVES < 8 ? WAVES : 8;  // FM > 4 keeps the partial tiles within 64 KiB
    switch (fm) {
    case 1: gemm_i8_skinny_pair<1, WAVES><<<nb, WAVES * 64, 0, st>>>(a1, a2, nb1); break;
    case 2: gemm_i8_skinny_pair<2, WAVES><<<nb, WAVES * 64, 0, st>>>(a1, a2, nb1); break;
    case 3: gemm_i8_skinny_pair<3, WAVES><<<nb, WAVES * 64, 0, st>>>(a1, a2, nb1); break;
    case 4: gemm_i8_skinny_pair<4, WAVES><<<nb, WAVES * 64, 0, st>>>(a1, a2, nb1); break;
    case 5: gemm_i8_skinny_pair<5, W8><<<nb, W8 * 64, 0, st>>>(a1, a2, nb1); break;
    case 6: gemm_i8_skinny_pair<6, W8><<<nb, W8 * 64, 0, st>>>(a1, a2, nb1); break;
    case 7: gemm_i8_skinny_pair<7, W8><<<nb, W8 * 64, 0, st>>>(a1, a2, nb1); break;
    default: gemm_i8_skinny_pair<8, W8><<<nb, W8 * 64, 0, st>>>(a1, a2, nb1); break;
    }
    VLA_LAUNCH_CHECK();
}

}  // namespace

// VLA_HIP_GEMM_PAIR=0 keeps every product in its own launch (read per call).
bool launch_gemm_i8_pair(const GemmArgs& a1, const GemmArgs& a2, hipStream_t st) {
    const char* e = std::getenv("VLA_HIP_GEMM_PAIR");
    if (e && e[0] == '0' && e[1] == '\0') return false;
    if (a1.M != a2.M || a1.N <= 0 || a2.N <= 0 || a1.K <= 0 || a2.K <= 0 || a1.K > kMaxI8K || a2.K > kMaxI8K)
        return false;
    if (a1.act < 0 || a1.act > 3 || a2.act < 0 || a2.act > 3) return false;
    for (const GemmArgs* a : {&a1, &a2}) {
        if (!a->out || !a->wscale || !a->ascale || a->ldo < a->N || a->ldb < kpad4(a->K) ||
            (!a->a_panel && a->lda < kpad4(a->K)))
            return false;
        if (a->a_panel && a->M > kPanelMaxRows) return false;
        if (!plain_skinny(*a)) return false;
    }
    const bool mid = skinny_mid_rows(a1.M, a1.N, a1.a_panel);
    if (mid != skinny_mid_rows(a2.M, a2.N, a2.a_panel)) return false;
    const int W = skinny_waves(a1.K);
    if (W != skinny_waves(a2.K)) return false;
    // one row-group count for both: as for one product of N1 + N2 columns, but
    // with at most 4 fragments per block. ACT's encoder (302 rows, q | k 1024
    // + v 512 columns, K = 512) on MI355X, graph replays per forward, two
    // launches 0.3149 ms, one launch with 3 / 4 / 5 / 7 / 10 row groups (7 /
    // 5 / 4 / 3 / 2 fragments per block) 0.3152 / 0.3082 / 0.2998 / 0.3056 /
    // 0.3042 ms. VLA_HIP_PAIR_R=<groups> forces a count (read per call).
    const int nfrag = (a1.M + 15) / 16;
    int g = skinny_row_groups(a1.M, a1.N + a2.N, a1.K, 1);
    g = g < (nfrag + 3) / 4 ? (nfrag + 3) / 4 : g;
    if (const char* r = std::getenv("VLA_HIP_PAIR_R"); r && std::atoi(r) > 0) g = std::atoi(r);
    g = g > nfrag ? nfrag : g;
    if (mid) g = g < (nfrag + 7) / 8 ? (nfrag + 7) / 8 : g;
    const int fm = (nfrag + g - 1) / g, groups = (nfrag + fm - 1) / fm;
    if (W == 16) run_skinny_pair<16>(a1, a2, fm, groups, st);
    else if (W == 8) run_skinny_pair<8>(a1, a2, fm, groups, st);
    else run_skinny_pair<4>(a1, a2, fm, groups, st);
    return true;
}

size_t gemm_split_bytes(int M, int N, int K) {
    const SplitPlan p = split_plan(M, N, K);
    return p.S > 1 ? (size_t)p.S * M * N * 4 : 0;
}

int rowop_gemm_block_rows(int M, int N) { return 16 * rowop_group_fm(M, N); }

bool rowop_gemm_fits(int op, int M, int K) {
    if (op == 1 || op < 0 || op > 3) return false;
    if (M < 1 || M > kPanelMaxRows || K < 4 || K % 4 || K > 2048) return false;
    const int fm = rowop_fm(M);
    return rowop_lds_main(fm, K) + 16 * fm * 4 <= kRowopMaxLds;
}

static bool ranges_overlap(const void* p, size_t pn, const void* q, size_t qn) {
    const char *a = static_cast<const char*>(p), *b = static_cast<const char*>(q);
    return a < b + qn && b < a + pn;
}

void launch_gemm_i8_rowop(const RowQArgs& r, const GemmArgs& a, hipStream_t st) {
    VLA_REQUIRE(r.op == 0 || r.op == 2 || r.op == 3, "gemm_i8_rowop: the fused row ops are 0, 2 and 3");
    VLA_REQUIRE(r.rows == a.M && r.H == a.K, "gemm_i8_rowop: the row op's rows and width must be M and K");
    VLA_REQUIRE(rowop_gemm_fits(r.op, a.M, a.K),
                "gemm_i8_rowop: need 1 <= M <= 128, K a multiple of 4 in [4, 2048] and the panel within LDS");
    VLA_REQUIRE(!r.out && !r.add && !r.out2 && !r.q2, "gemm_i8_rowop: the fused row op has no fp32 or second output");
    VLA_REQUIRE(!r.q || (!r.q_panel && r.qs && r.ldq >= kpad4(a.K) && r.ldq % 4 == 0 && aligned(r.q, 4)),
                "gemm_i8_rowop: the quantized-row copy is row-major, 4-byte aligned, ldq >= i8_kpad(K), with scales");
    VLA_REQUIRE(r.x && (r.ldx >= a.K || (r.taps && r.ldx > 0)) && r.ldx % 4 == 0 && aligned(r.x, 16),
                "gemm_i8_rowop: x rows must be 16-byte aligned");
    VLA_REQUIRE(r.op == 0 || r.op == 3 || (r.w && aligned(r.w, 16) && (!r.b || aligned(r.b, 16))),
                "gemm_i8_rowop: norm weights must be 16-byte aligned");
    VLA_REQUIRE(r.op != 3 || (r.u && r.ldu >= a.K && r.ldu % 4 == 0 && aligned(r.u, 16)),
                "gemm_i8_rowop: silu_gate needs 16-byte aligned u rows");
    VLA_REQUIRE(a.N > 0 && a.K <= kMaxI8K && a.B && a.ldb >= kpad4(a.K) && a.ldb % 16 == 0 && aligned(a.B, 16),
                "gemm_i8_rowop: weights must be 16-byte aligned rows of stride >= i8_kpad(K)");
    VLA_REQUIRE(a.out && a.wscale && a.ldo >= a.N && !a.acc32, "gemm_i8_rowop: needs out, wscale and ldo >= N");
    VLA_REQUIRE(a.act >= 0 && a.act <= 3, "gemm_i8_rowop: unknown activation");
    const size_t ob = ((size_t)(a.M - 1) * a.ldo + a.N) * sizeof(float);
    VLA_REQUIRE(!ranges_overlap(a.out, ob, r.x, ((size_t)(a.M - 1) * r.ldx + a.K) * sizeof(float)) &&
                    (r.op != 3 || !ranges_overlap(a.out, ob, r.u, ((size_t)(a.M - 1) * r.ldu + a.K) * sizeof(float))),
                "gemm_i8_rowop: out must not overlap the rows the row op reads");
    if (r.op == 0) run_rowop_nv<0>(r, a, st);
    else if (r.op == 2) run_rowop_nv<2>(r, a, st);
    else run_rowop_nv<3>(r, a, st);
}

}  // namespace hip
}  // namespace vla
