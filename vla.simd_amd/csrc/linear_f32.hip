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
// the column reads of the fragment loads do not collide on a bank).

#include "act.h"
#include "common.h"

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

}  // namespace

void launch_linear_f32(float* out, int ldo, const float* x, int ldx, const float* W, int ldw,
                       const float* bias, int M, int N, int K, int act, int accumulate, float alpha,
                       hipStream_t st) {
    VLA_REQUIRE(M >= 0 && N > 0 && K > 0, "linear_f32: need M >= 0, N > 0, K > 0");
    VLA_REQUIRE(ldx >= K && ldw >= K && ldo >= N, "linear_f32: row strides shorter than the rows");
    VLA_REQUIRE(out && x && W, "linear_f32: null buffer");
    VLA_REQUIRE(act >= 0 && act <= 4, "linear_f32: unknown activation");
    if (M == 0) return;
    // small grids (the batch-1 action heads) take 32 x 32 tiles so more CUs get work
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

}  // namespace hip
}  // namespace vla
