// linear_f32.hip - fp32 linear layers on the fp32 matrix cores (gfx950).
//
// out[m, n] (+)= act(sum_k x[m, k] * W[n, k] + bias[n])
//
// The layers the reference keeps in fp32 around the int8 path go through this
// kernel: Linear::Role::Generic (dense_linear, src/hal/common/gemm.cpp) and the
// Gemm-role layers a model leaves out of its int8 mask - ACT's state_proj and
// action head (src/models/act/act_transformer.cpp:127-128), Octo's token
// projections outside OCTO_INT8 bit 8 (src/models/octo/octo_transformer.cpp:60-62),
// SmolVLA's flow-matching projections (src/models/smolvla/action_expert.cpp:196-211).
// fp32 results differ from the reference's only by summation order.
//
// v_mfma_f32_16x16x4f32: lane l supplies A[row l % 16][k l / 16] and
// B[col l % 16][k l / 16]; output lane l holds column l % 16, rows
// 4 * (l / 16) + r. A block owns a BM x BN tile with four waves in a 2 x 2 grid;
// K advances in 16-wide slabs staged through LDS (rows padded by one float so
// the column reads of the fragment loads do not collide on a bank). M <= 128
// takes a split-K kernel instead (see linear_f32_skinny).

#include "act.h"
#include "common.h"

#include <cstdlib>

#pragma clang fp contract(off)

namespace vla {
namespace hip {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

template <int BM, int BN>
__global__ __launch_bounds__(256) void linear_f32_kernel(float* __restrict__ out, int ldo,
                                                         const float* __restrict__ x, int ldx,
                                                         const float* __restrict__ W, int ldw,
                                                         const float* __restrict__ bias, int M,
                                                         int N, int K, int act, int accumulate,
                                                         float alpha) {
    constexpr int BK = 16, SP = BK + 1;
    constexpr int TM = BM / 2, TN = BN / 2, FM = TM / 16, FN = TN / 16;
    __shared__ float sa[BM * SP], sb[BN * SP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

    v4f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    for (int k0 = 0; k0 < K; k0 += BK) {
        for (int e = tid; e < BM * BK; e += 256) {
            const int r = e / BK, c = e % BK, m = m0 + r, k = k0 + c;
            sa[r * SP + c] = (m < M && k < K) ? x[(size_t)m * ldx + k] : 0.0f;
        }
        for (int e = tid; e < BN * BK; e += 256) {
            const int r = e / BK, c = e % BK, n = n0 + r, k = k0 + c;
            sb[r * SP + c] = (n < N && k < K) ? W[(size_t)n * ldw + k] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int ks = 0; ks < BK; ks += 4) {
            float af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; i++) af[i] = sa[(wm * TM + i * 16 + (lane & 15)) * SP + ks + (lane >> 4)];
#pragma unroll
            for (int j = 0; j < FN; j++) bf[j] = sb[(wn * TN + j * 16 + (lane & 15)) * SP + ks + (lane >> 4)];
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }

#pragma unroll
    for (int j = 0; j < FN; j++) {
        const int n = n0 + wn * TN + j * 16 + (lane & 15);
        if (n >= N) continue;
        const float b = bias ? bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm * TM + i * 16 + 4 * (lane >> 4) + r;
                if (m >= M) continue;
                float v = acc[i][j][r] + b;
                switch (act) {
                case 1: v = act_relu(v); break;
                case 2: v = act_gelu_tanh(v); break;
                case 3: v = act_gelu_erf(v); break;
                case 4: v = act_silu(v); break;
                default: break;
                }
                float* o = out + (size_t)m * ldo + n;
                *o = accumulate ? fmaf(alpha, v, *o) : v;
            }
    }
}

// The tiled form for M > 128 with 16-byte aligned rows (the conv GEMMs of
// ACT's fp32 backbone and Octo's stems, the big fp32 projections): BM x BN
// tiles, four waves in a 2 x 2 grid, 32-wide K slabs loaded as float4 runs
// (coalesced 128-byte row segments) into registers while the previous slab
// computes from the other LDS buffer. Within a 16-wide k chunk, lane group g
// feeds k = 4g + t to the t-th of four MFMAs (the same order for A and B, so
// each MFMA still sums matching products), which lets a lane read its four
// A (or B) values as one ds_read_b128; LDS rows are padded to BK + 4 floats,
// so the 16 rows one read touches fall on distinct banks.
// CONV: x is an NHWC map and row m of A is output pixel m's k x k patch,
// column (ky * k + kx) * Cin + ci (im2col's order), gathered by the A loads
// themselves: with Cin % 32 == 0 a thread's float4 of a 32-wide slab always
// lies in one tap, and its tap advances by 32 channels per slab. Same
// products in the same order as im2col + this kernel; no column matrix.
struct ConvGeom {
    int H, Wd, Cin, k, stride, pad, Wout;
};

template <int BM, int BN, bool CONV = false>
__global__ __launch_bounds__(256) void linear_f32_tiled(float* __restrict__ out, int ldo,
                                                        const float* __restrict__ x, int ldx,
                                                        const float* __restrict__ W, int ldw,
                                                        const float* __restrict__ bias, int M, int N,
                                                        int K, int act, int accumulate, float alpha,
                                                        ConvGeom cg, float* __restrict__ part, int kchunk) {
    constexpr int BK = 32, SP = BK + 4;
    constexpr int TM = BM / 2, TN = BN / 2, FM = TM / 16, FN = TN / 16;
    constexpr int AV = BM * BK / 4 / 256, BV = BN * BK / 4 / 256;  // float4 loads per thread
    static_assert(AV >= 1 && BV >= 1 && TM % 16 == 0 && TN % 16 == 0, "tile");
    __shared__ __attribute__((aligned(16))) float sm[2][(BM + BN) * SP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    // split K (part != null): chunk blockIdx.z of kchunk columns, raw sums into
    // its slice of part; K becomes the chunk's length
    const int kbeg = part ? blockIdx.z * kchunk : 0;
    if (part) K = K - kbeg < kchunk ? K - kbeg : kchunk;

    // float4 v of a slab: row v / 8, k 4 (v % 8); rows past the matrix clamped
    const float* ap[AV];
    const float* bp[BV];
    int ao[AV], bo[BV], kk[AV > BV ? AV : BV];
    int iy0[AV], ix0[AV];  // CONV: the patch origin of each loaded row
#pragma unroll
    for (int j = 0; j < AV; j++) {
        const int v = tid + 256 * j, r = v >> 3, k = (v & 7) * 4;
        const int m = m0 + r < M ? m0 + r : M - 1;
        if (CONV) {
            const int oy = m / cg.Wout, ox = m - oy * cg.Wout;
            iy0[j] = oy * cg.stride - cg.pad;
            ix0[j] = ox * cg.stride - cg.pad;
            ap[j] = x;
        } else {
            ap[j] = x + (size_t)m * ldx + kbeg + k;
        }
        ao[j] = r * SP + k;
    }
#pragma unroll
    for (int j = 0; j < BV; j++) {
        const int v = tid + 256 * j, r = v >> 3, k = (v & 7) * 4;
        const int n = n0 + r < N ? n0 + r : N - 1;
        bp[j] = W + (size_t)n * ldw + kbeg + k;
        bo[j] = (BM + r) * SP + k;
    }
    const int kq = (tid & 7) * 4;  // this thread's k offset within a slab (same for every load)
    (void)kk;
    float4 ra[AV], rb[BV];
    auto ld4 = [&](const float* p, int k) {
        if (k + 4 <= K) return *reinterpret_cast<const float4*>(p);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (k < K) v.x = p[0];
        if (k + 1 < K) v.y = p[1];
        if (k + 2 < K) v.z = p[2];
        return v;  // k + 3 >= K here
    };
    // CONV: the tap of this thread's next A slab (kbeg is a multiple of 32)
    int ci = kq, kx = 0, ky = 0;
    if (CONV && kbeg) {
        const int t = kbeg / cg.Cin;
        ci = kbeg - t * cg.Cin + kq;
        ky = t / cg.k;
        kx = t - ky * cg.k;
    }
    auto gload = [&](int k0) {
        if (CONV) {  // called for k0 = 0, BK, 2 BK, ... in order
#pragma unroll
            for (int j = 0; j < AV; j++) {
                const int iy = iy0[j] + ky, ix = ix0[j] + kx;
                ra[j] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (iy >= 0 && iy < cg.H && ix >= 0 && ix < cg.Wd)
                    ra[j] = *reinterpret_cast<const float4*>(x + ((size_t)iy * cg.Wd + ix) * cg.Cin + ci);
            }
            ci += BK;
            if (ci >= cg.Cin) {
                ci -= cg.Cin;
                if (++kx == cg.k) {
                    kx = 0;
                    ++ky;
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < AV; j++) ra[j] = ld4(ap[j] + k0, k0 + kq);
        }
#pragma unroll
        for (int j = 0; j < BV; j++) rb[j] = ld4(bp[j] + k0, k0 + kq);
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int j = 0; j < AV; j++) *reinterpret_cast<float4*>(&sm[buf][ao[j]]) = ra[j];
#pragma unroll
        for (int j = 0; j < BV; j++) *reinterpret_cast<float4*>(&sm[buf][bo[j]]) = rb[j];
    };

    v4f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
    const int r16 = lane & 15, g4 = (lane >> 4) * 4;
    auto compute = [&](int buf) {
        const float* s = sm[buf];
#pragma unroll
        for (int kc = 0; kc < BK; kc += 16) {
            float4 af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; i++)
                af[i] = *reinterpret_cast<const float4*>(s + (wm * TM + i * 16 + r16) * SP + kc + g4);
#pragma unroll
            for (int j = 0; j < FN; j++)
                bf[j] = *reinterpret_cast<const float4*>(s + (BM + wn * TN + j * 16 + r16) * SP + kc + g4);
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i].x, bf[j].x, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i].y, bf[j].y, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i].z, bf[j].z, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i].w, bf[j].w, acc[i][j], 0, 0, 0);
                }
        }
    };

    const int nk = (K + BK - 1) / BK;
    gload(0);
    lstore(0);
    if (nk > 1) gload(BK);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        compute(buf);
        if (kt + 1 < nk) {
            lstore(buf ^ 1);  // slab kt + 1, loaded during this compute
            if (kt + 2 < nk) gload((kt + 2) * BK);
        }
        __syncthreads();
    }

    if (part) {
        float* pz = part + (size_t)blockIdx.z * M * N;
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int n = n0 + wn * TN + j * 16 + r16;
            if (n >= N) continue;
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = m0 + wm * TM + i * 16 + g4 + r;
                    if (m < M) pz[(size_t)m * N + n] = acc[i][j][r];
                }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < FN; j++) {
        const int n = n0 + wn * TN + j * 16 + r16;
        if (n >= N) continue;
        const float b = bias ? bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm * TM + i * 16 + g4 + r;
                if (m >= M) continue;
                float v = acc[i][j][r] + b;
                switch (act) {
                case 1: v = act_relu(v); break;
                case 2: v = act_gelu_tanh(v); break;
                case 3: v = act_gelu_erf(v); break;
                case 4: v = act_silu(v); break;
                default: break;
                }
                float* o = out + (size_t)m * ldo + n;
                *o = accumulate ? fmaf(alpha, v, *o) : v;
            }
    }
}

// M <= 128 (the batch-1 action heads and flow-matching projections): a block
// owns 16 output columns and every row; its W waves split K in 16-wide steps
// and read their MFMA operands straight from global memory as float4 runs
// (lane group g takes k = 4g .. 4g+3 of a step; A and B use the same k order,
// so each MFMA still sums matching products). The waves' partial sums meet in
// LDS before the epilogue.
template <int FM, int W, bool VEC>
__global__ __launch_bounds__(W * 64) void linear_f32_skinny(float* __restrict__ out, int ldo,
                                                            const float* __restrict__ x, int ldx,
                                                            const float* __restrict__ Wt, int ldw,
                                                            const float* __restrict__ bias, int M,
                                                            int N, int K, int act, int accumulate,
                                                            float alpha) {
    __shared__ float red[W * FM * 256];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * 16, mb = blockIdx.y * 16 * FM;  // row tile blockIdx.y of 16 * FM rows
    const int n = n0 + c < N ? n0 + c : N - 1;
    const float* brow = Wt + (size_t)n * ldw;
    const float* arow[FM];
#pragma unroll
    for (int i = 0; i < FM; i++) {
        const int m = mb + 16 * i + c < M ? mb + 16 * i + c : M - 1;
        arow[i] = x + (size_t)m * ldx;
    }
    auto load4 = [&](const float* row, int k) {
        if (VEC && k + 4 <= K) return *reinterpret_cast<const float4*>(row + k);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (k < K) v.x = row[k];
        if (k + 1 < K) v.y = row[k + 1];
        if (k + 2 < K) v.z = row[k + 2];
        if (k + 3 < K) v.w = row[k + 3];
        return v;
    };
    v4f acc[FM];
#pragma unroll
    for (int i = 0; i < FM; i++) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};
    // P of the wave's K steps per round: all their loads are issued before the
    // first MFMA (one wait per round instead of one per step); the MFMAs run
    // in the same step order, so the sums are the same
    constexpr int P = FM <= 4 ? 4 : 2;
    for (int k16r = wave * 16; k16r < K; k16r += P * W * 16) {
        float4 b[P], a[P][FM];
#pragma unroll
        for (int p = 0; p < P; p++) {
            const int k16 = k16r + p * W * 16;
            if (k16 < K) {  // wave-uniform
                const int k = k16 + 4 * g;
                b[p] = load4(brow, k);
#pragma unroll
                for (int i = 0; i < FM; i++) a[p][i] = load4(arow[i], k);
            }
        }
#pragma unroll
        for (int p = 0; p < P; p++) {
            if (k16r + p * W * 16 < K) {
#pragma unroll
                for (int i = 0; i < FM; i++) {
                    acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[p][i].x, b[p].x, acc[i], 0, 0, 0);
                    acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[p][i].y, b[p].y, acc[i], 0, 0, 0);
                    acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[p][i].z, b[p].z, acc[i], 0, 0, 0);
                    acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[p][i].w, b[p].w, acc[i], 0, 0, 0);
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) red[((wave * FM + i) * 4 + r) * 64 + lane] = acc[i][r];
    __syncthreads();
    // thread e sums element e of the FM x 4 x 64 lane-major tile over the waves
    for (int e = tid; e < FM * 256; e += W * 64) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < W; w++) v += red[w * FM * 256 + e];
        const int l = e & 63, r = (e >> 6) & 3, i = e >> 8;
        const int m = mb + 16 * i + 4 * (l >> 4) + r, nn = n0 + (l & 15);
        if (m >= M || nn >= N) continue;
        v = v + (bias ? bias[nn] : 0.0f);
        switch (act) {
        case 1: v = act_relu(v); break;
        case 2: v = act_gelu_tanh(v); break;
        case 3: v = act_gelu_erf(v); break;
        case 4: v = act_silu(v); break;
        default: break;
        }
        float* o = out + (size_t)m * ldo + nn;
        *o = accumulate ? fmaf(alpha, v, *o) : v;
    }
}

template <int FM, bool VEC>
void launch_skinny_fm(float* out, int ldo, const float* x, int ldx, const float* W, int ldw,
                      const float* bias, int M, int N, int K, int act, int accumulate, float alpha,
                      hipStream_t st) {
    const int steps = (K + 15) / 16;
    // row groups of 16 * FM rows (grid.y): as the int8 skinny GEMM, the fewest
    // that give every CU a block; each output's sum is unchanged
    const dim3 blocks((N + 15) / 16, (M + 16 * FM - 1) / (16 * FM));
    // about four K steps per wave, at most 8 waves
    const int w = steps >= 32 ? 8 : steps >= 16 ? 4 : steps >= 8 ? 2 : 1;
    switch (w) {
    case 8: linear_f32_skinny<FM, 8, VEC><<<blocks, 512, 0, st>>>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act, accumulate, alpha); break;
    case 4: linear_f32_skinny<FM, 4, VEC><<<blocks, 256, 0, st>>>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act, accumulate, alpha); break;
    case 2: linear_f32_skinny<FM, 2, VEC><<<blocks, 128, 0, st>>>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act, accumulate, alpha); break;
    default: linear_f32_skinny<FM, 1, VEC><<<blocks, 64, 0, st>>>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act, accumulate, alpha); break;
    }
}

template <bool VEC>
void launch_skinny(float* out, int ldo, const float* x, int ldx, const float* W, int ldw,
                   const float* bias, int M, int N, int K, int act, int accumulate, float alpha,
                   hipStream_t st) {
    const int nfrag = (M + 15) / 16, nb = (N + 15) / 16;
    int g = (256 + nb - 1) / nb;  // 256 CUs
    if (const char* e = std::getenv("VLA_HIP_SKINNY_R")) g = *e ? std::atoi(e) : g;
    g = g < 1 ? 1 : g > nfrag ? nfrag : g;
    switch ((nfrag + g - 1) / g) {
    case 1: launch_skinny_fm<1, VEC>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act, accumulate, alpha, st); break;
    case 2: launch_skinny_fm<2, VEC>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act, accumulate, alpha, st); break;
    case 3: launch_skinny_fm<3, VEC>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act, accumulate, alpha, st); break;
    case 4: launch_skinny_fm<4, VEC>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act, accumulate, alpha, st); break;
    case 5: launch_skinny_fm<5, VEC>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act, accumulate, alpha, st); break;
    case 6: launch_skinny_fm<6, VEC>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act, accumulate, alpha, st); break;
    case 7: launch_skinny_fm<7, VEC>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act, accumulate, alpha, st); break;
    default: launch_skinny_fm<8, VEC>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act, accumulate, alpha, st); break;
    }
}

// The split-K partial sums of linear_f32_tiled: out = act(sum_z part[z] + bias)
// with the chunks added in z order, then the epilogue of the unsplit kernel.
__global__ __launch_bounds__(256) void linear_f32_split_reduce(float* __restrict__ out, int ldo,
                                                               const float* __restrict__ part, int S, int M, int N,
                                                               const float* __restrict__ bias, int act,
                                                               int accumulate, float alpha) {
    const int64_t MN = (int64_t)M * N;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < MN; e += (int64_t)gridDim.x * blockDim.x) {
        float v = part[e];
        for (int z = 1; z < S; z++) v += part[z * MN + e];
        const int m = (int)(e / N), n = (int)(e - (int64_t)m * N);
        v = v + (bias ? bias[n] : 0.0f);
        switch (act) {
        case 1: v = act_relu(v); break;
        case 2: v = act_gelu_tanh(v); break;
        case 3: v = act_gelu_erf(v); break;
        case 4: v = act_silu(v); break;
        default: break;
        }
        float* o = out + (size_t)m * ldo + n;
        *o = accumulate ? fmaf(alpha, v, *o) : v;
    }
}

constexpr int kCUs = 256;  // MI355X compute units

// Split-K plan for M > 128 over K >= 1024 when 64 x 64 tiles number < 128
// (ResNet's last stages): S chunks of K (multiples of 32, >= 256) so that
// S x tiles reaches about two blocks per CU, S <= 8.
struct F32Split {
    int S = 1, kchunk = 0;
};
// VLA_HIP_F32_SMALL_TILES=0 keeps 64 x 64 tiles for few-tile fp32 layers
// (read per call; A/B runs)
static bool f32_small_tiles_on() {
    const char* e = std::getenv("VLA_HIP_F32_SMALL_TILES");
    return !(e && e[0] == '0' && e[1] == '\0');
}

F32Split f32_split_plan(int M, int N, int K) {
    F32Split p;
    const long t64 = (long)((M + 63) / 64) * ((N + 63) / 64);
    if (M <= 128 || t64 >= 128 || K < 1024) return p;
    int S = (int)((2 * kCUs + t64 - 1) / t64);
    S = S < 8 ? S : 8;
    int kc = ((K + S - 1) / S + 31) / 32 * 32;
    kc = kc > 256 ? kc : 256;
    p.S = (K + kc - 1) / kc;
    p.kchunk = kc;
    if (p.S < 2) p = F32Split{};
    return p;
}

void launch_f32_split(float* out, int ldo, const float* x, int ldx, const float* W, int ldw, const float* bias,
                      int M, int N, int K, int act, int accumulate, float alpha, const ConvGeom& cg, bool conv,
                      const F32Split& p, float* part, hipStream_t st) {
    const dim3 grid((N + 63) / 64, (M + 63) / 64, p.S);
    if (conv)
        linear_f32_tiled<64, 64, true><<<grid, 256, 0, st>>>(out, ldo, x, ldx, W, ldw, bias, M, N, K, 0, 0, 1.0f, cg,
                                                             part, p.kchunk);
    else
        linear_f32_tiled<64, 64><<<grid, 256, 0, st>>>(out, ldo, x, ldx, W, ldw, bias, M, N, K, 0, 0, 1.0f, cg, part,
                                                       p.kchunk);
    VLA_LAUNCH_CHECK();
    const int64_t MN = (int64_t)M * N;
    const int blocks = (int)((MN + 255) / 256 < 4096 ? (MN + 255) / 256 : 4096);
    linear_f32_split_reduce<<<blocks, 256, 0, st>>>(out, ldo, part, p.S, M, N, bias, act, accumulate, alpha);
    VLA_LAUNCH_CHECK();
}

// VLA_F32_TILED=0 keeps the LDS-scalar kernel (A/B comparisons)
bool env_off_f32tiled() {
    const char* e = std::getenv("VLA_F32_TILED");
    return e && e[0] == '0' && e[1] == '\0';
}

}  // namespace

size_t linear_f32_split_floats(int M, int N, int K) {
    const F32Split p = f32_split_plan(M, N, K);
    return p.S > 1 ? (size_t)p.S * M * N : 0;
}

void launch_linear_f32(float* out, int ldo, const float* x, int ldx, const float* W, int ldw,
                       const float* bias, int M, int N, int K, int act, int accumulate, float alpha,
                       hipStream_t st, float* work, size_t work_floats, bool taps) {
    VLA_REQUIRE(M >= 0 && N > 0 && K > 0, "linear_f32: need M >= 0, N > 0, K > 0");
    VLA_REQUIRE((ldx >= K || (taps && ldx > 0)) && ldw >= K && ldo >= N,
                "linear_f32: row strides shorter than the rows");
    VLA_REQUIRE(out && x && W, "linear_f32: null buffer");
    VLA_REQUIRE(act >= 0 && act <= 4, "linear_f32: unknown activation");
    if (M == 0) return;
    if (M <= 128) {
        const bool vec = ldx % 4 == 0 && ldw % 4 == 0 && aligned(x, 16) && aligned(W, 16);
        if (vec) launch_skinny<true>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act, accumulate, alpha, st);
        else launch_skinny<false>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act, accumulate, alpha, st);
        VLA_LAUNCH_CHECK();
        return;
    }
    if (ldx % 4 == 0 && ldw % 4 == 0 && aligned(x, 16) && aligned(W, 16) && !env_off_f32tiled()) {
        const long t64 = (long)((M + 63) / 64) * ((N + 63) / 64);
        const F32Split sp = f32_split_plan(M, N, K);
        if (sp.S > 1 && work && work_floats >= (size_t)sp.S * M * N && aligned(work, 16)) {
            // few tiles over a long K with a workspace: 64 x 64 tiles split over K
            launch_f32_split(out, ldo, x, ldx, W, ldw, bias, M, N, K, act, accumulate, alpha, ConvGeom{}, false, sp,
                             work, st);
            return;
        }
        if (t64 < 128 && K >= 1024) {
            // few tiles over a long K (ResNet's last stages): the split-K form,
            // 64-row x 16-column blocks whose 8 waves share K, so the chain of
            // dependent loads per wave is an eighth of K
            const dim3 grid((N + 15) / 16, (M + 63) / 64);
            linear_f32_skinny<4, 8, true><<<grid, 512, 0, st>>>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act,
                                                                 accumulate, alpha);
            VLA_LAUNCH_CHECK();
            return;
        }
        // 128 x 64 tiles when they still give every CU work, 64 x 64 from 128
        // such tiles, else 32 x 32 (a fourth of the fp32 matrix work per
        // block: Octo's 256 x 768 x 512 token projections, 48 tiles of 64 x
        // 64, were ~20 us each, one fp32 MFMA chain of a whole tile per CU)
        const long t128 = (long)((M + 127) / 128) * ((N + 63) / 64);
        if (t128 >= 256) {
            const dim3 grid((N + 63) / 64, (M + 127) / 128);
            linear_f32_tiled<128, 64><<<grid, 256, 0, st>>>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act,
                                                            accumulate, alpha, ConvGeom{}, nullptr, 0);
        } else if (t64 < 128 && f32_small_tiles_on()) {
            const dim3 grid((N + 31) / 32, (M + 31) / 32);
            linear_f32_tiled<32, 32><<<grid, 256, 0, st>>>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act,
                                                           accumulate, alpha, ConvGeom{}, nullptr, 0);
        } else {
            const dim3 grid((N + 63) / 64, (M + 63) / 64);
            linear_f32_tiled<64, 64><<<grid, 256, 0, st>>>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act,
                                                           accumulate, alpha, ConvGeom{}, nullptr, 0);
        }
        VLA_LAUNCH_CHECK();
        return;
    }
    // small grids take 32 x 32 tiles so more CUs get work
    const long big = (long)((M + 63) / 64) * ((N + 63) / 64);
    if (big >= 128) {
        const dim3 grid((N + 63) / 64, (M + 63) / 64);
        linear_f32_kernel<64, 64><<<grid, 256, 0, st>>>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act,
                                                        accumulate, alpha);
    } else {
        const dim3 grid((N + 31) / 32, (M + 31) / 32);
        linear_f32_kernel<32, 32><<<grid, 256, 0, st>>>(out, ldo, x, ldx, W, ldw, bias, M, N, K, act,
                                                        accumulate, alpha);
    }
    VLA_LAUNCH_CHECK();
}

bool launch_conv_f32_implicit(float* out, const float* x, int H, int Wd, int Cin, int k, int stride, int pad,
                              int Hout, int Wout, const float* W, const float* bias, int Cout, int act,
                              hipStream_t st, float* work, size_t work_floats) {
    const char* e = std::getenv("VLA_CONV_F32_IMPLICIT");  // 0: im2col + GEMM (A/B runs)
    if (e && e[0] == '0' && e[1] == '\0') return false;
    VLA_REQUIRE(out && x && W && H > 0 && Wd > 0 && Cin > 0 && k > 0 && stride > 0 && pad >= 0 && Cout > 0 &&
                    Hout > 0 && Wout > 0 && act >= 0 && act <= 4,
                "conv_f32: bad arguments");
    const int64_t K64 = (int64_t)k * k * Cin, M64 = (int64_t)Hout * Wout;
    // the output pixels' patches stay inside the padded input
    VLA_REQUIRE((int64_t)(Hout - 1) * stride + k <= (int64_t)H + 2 * pad &&
                    (int64_t)(Wout - 1) * stride + k <= (int64_t)Wd + 2 * pad,
                "conv_f32: output larger than the padded input allows");
    if (Cin % 32 || K64 > INT32_MAX || M64 > INT32_MAX || (int64_t)H * Wd * Cin > INT32_MAX) return false;
    if (!aligned(x, 16) || !aligned(W, 16) || env_off_f32tiled()) return false;
    const int M = (int)M64, K = (int)K64, N = Cout;
    if (M <= 128) return false;
    const long t64 = (long)((M + 63) / 64) * ((N + 63) / 64);
    const ConvGeom cg{H, Wd, Cin, k, stride, pad, Wout};
    const F32Split sp = f32_split_plan(M, N, K);
    if (sp.S > 1) {  // as launch_linear_f32: split over K with a workspace, else not here
        if (!(work && work_floats >= (size_t)sp.S * M * N && aligned(work, 16))) return false;
        launch_f32_split(out, N, x, K, W, K, bias, M, N, K, act, 0, 1.0f, cg, true, sp, work, st);
        return true;
    }
    if (t64 < 128 && K >= 1024) return false;  // the skinny route of launch_linear_f32
    const long t128 = (long)((M + 127) / 128) * ((N + 63) / 64);
    if (t128 >= 256) {
        const dim3 grid((N + 63) / 64, (M + 127) / 128);
        linear_f32_tiled<128, 64, true><<<grid, 256, 0, st>>>(out, N, x, K, W, K, bias, M, N, K, act, 0, 1.0f, cg,
                                                              nullptr, 0);
    } else {
        const dim3 grid((N + 63) / 64, (M + 63) / 64);
        linear_f32_tiled<64, 64, true><<<grid, 256, 0, st>>>(out, N, x, K, W, K, bias, M, N, K, act, 0, 1.0f, cg,
                                                             nullptr, 0);
    }
    VLA_LAUNCH_CHECK();
    return true;
}

}  // namespace hip
}  // namespace vla
