// attn.hip - fused masked GQA attention (QK^T -> online softmax -> PV) on gfx950.
//
// Semantics are the reference's gqa_attention_masked (src/ops/lm_ops.h:33;
// scalar reference src/hal/scalar/attn.cpp:22-87, AVX2 engine
// src/hal/avx2/attn.cpp:266-447):
//   score = (q . k) * scale + mask;  a key whose mask entry is lowest() or whose
//   score is -inf gets weight exactly 0;  out = sum_j softmax_j * v_j;  a row
//   with every key blocked is the uniform mean of V over all seq_k keys
//   (attn_uniform_row, avx2/attn.cpp:45-52).
// fp32 throughout; results are tolerance-class against the reference (its exp
// is a Cephes polynomial, its sums run in another order).
//
// A block owns 16 queries of one head; its W waves split the key range: wave w
// takes key tiles w, w + W, ... (KT keys each), stages each tile in its own
// LDS region (no block barrier in the main loop) and keeps its own online
// softmax state; at the end the waves merge their (max, sum, output) through
// LDS. Small problems (the batch-1 action chunks) thereby still occupy many
// waves, and large ones get W-fold more waves than query tiles.
// Both products run on the fp32 matrix cores (v_mfma_f32_16x16x4_f32, one
// float per lane per operand):
//   S^T = K Q^T : A = K tile rows (keys), B = Q^T; lane l's result holds
//                 S[q = l%16][key = 16*kt + 4*(l/16) + r], r = 0..3;
//   O^T = V^T P^T: A = V^T, B = P^T. The B operand lane l must supply is
//                 P[q = l%16][key = 16*kt + 4*(l/16) + r] - exactly the value
//                 lane l already holds from S^T, so P never moves between lanes.
// The head dimension is walked as d = g*(HDP/4) + s for lane group g = l/16,
// so each lane's Q slice and each K row read are contiguous (ds_read_b128).
// LDS rows are HDP+4 floats: the 16 rows of one read land on distinct banks,
// and the four lane groups of a V read land 16 banks apart. The next tile's
// K/V rows are loaded into registers while the current tile computes.
// Scores and the running max stay in the natural domain (dot*scale + mask, as
// the reference forms them); exp(x) is evaluated as v_exp_f32(x * log2 e).

#include "common.h"

#include <cfloat>
#include <cstdlib>

namespace vla {
namespace hip {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.44269504088896340736f;

__device__ __forceinline__ v4f mfma_f32(float a, float b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max / sum of x over the lanes l, l^16, l^32, l^48 (the four 16-lane rows of
// a wave) with gfx950's row-swap permutes, VALU ops instead of LDS round trips.
// permlane16_swap(x, x) returns, in every lane, the values of the lane pair
// {l, l^16} (one from the even row, one from the odd row); permlane32_swap the
// pair {l, l^32}. The sum adds each pair in either order, which is the same
// float: the results equal those of x op shfl_xor(x, 16), then 32.
__device__ __forceinline__ float rows_max(float x) {
    const unsigned u = __float_as_uint(x);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const unsigned v = __float_as_uint(y);
    const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
    const unsigned u = __float_as_uint(x);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const unsigned v = __float_as_uint(y);
    const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Orders this wave's LDS accesses (its writes before other lanes' reads) with
// no block barrier.
__device__ __forceinline__ void wave_lds_sync() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4));  // lgkmcnt(0) only
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
}

template <int HDP, int KT, int W>
struct AttnCfg {
    static constexpr int SK = HDP + 4;               // LDS row, floats
    static constexpr int TILE = 2 * KT * SK;         // K + V of one wave, floats
    static constexpr int F4 = KT * HDP / 4 / 64;     // float4 loads per lane per K (or V) tile
    static constexpr int MO = HDP + 4;               // merge row, floats: the 16 rows of one
                                                     // float4 access fall on distinct banks
    static constexpr int MERGE = W * (32 + 16 * MO);
    static constexpr int MAIN = 4 * (W * TILE > MERGE ? W * TILE : MERGE);  // bytes
    static constexpr int ALLOW = 4096;  // group table bytes kept in LDS (n_groups <= 64)
    static constexpr int LDS = MAIN + ALLOW;
    static_assert(KT % 16 == 0 && (KT * HDP / 4) % 64 == 0, "tile shape");
};

// MKC: the mask class compiled in - 1 dense, 3 group table (per-key data
// prefetched with each tile), 0 for kinds 0 and 2 (none, causal), which read
// no per-key data.
template <int HDP, int KT, int W, int MKC>
__global__ __launch_bounds__(W * 64) void attn_fwd(AttnArgs a) {
    constexpr bool KD = MKC != 0;
    using C = AttnCfg<HDP, KT, W>;
    constexpr int SK = C::SK, F4 = C::F4;
    constexpr int NT = KT / 16;
    constexpr int QS = HDP / 4;
    constexpr int DT = HDP / 16;
    extern __shared__ __attribute__((aligned(16))) float smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    // XCD-aware block order for grids of at most one round (256 blocks; ACT,
    // SmolVLA): the hardware deals workgroup i to XCD i % 8, so each XCD is
    // given a contiguous run of (head, query tile) pairs and its L2 holds the
    // K/V rows of a few heads instead of every head's. Larger grids (Octo,
    // SigLIP) measured slower that way; they take the balanced order below.
    const int nqt = gridDim.x, total = nqt * gridDim.y;
    const int bid = blockIdx.y * nqt + blockIdx.x;
    int qt, h;
    if (total <= 256) {
        const int xcd = bid & 7, per = total >> 3, rem = total & 7;
        const int logical = xcd * per + (xcd < rem ? xcd : rem) + (bid >> 3);
        qt = logical % nqt;
        h = logical / nqt;
    } else if constexpr (W <= 4) {
        // grids of 1.5+ blocks per CU take 4 waves per block (run_attn). Rounds
        // of 256 blocks put one block on every CU (block b and b + 256 share a
        // CU); under causal and block-causal masks a query tile's work grows
        // with its index, so tiles are dealt heaviest first with every other
        // round reversed: a CU's heavy block meets a light one, and a last
        // partial round gets the lightest
        const int r = bid >> 8, p = bid & 255, start = r << 8;
        const int len = total - start < 256 ? total - start : 256;
        const int i = total - 1 - (start + ((r & 1) ? len - 1 - p : p));
        qt = i / gridDim.y;
        h = i - qt * gridDim.y;
    } else {
        qt = bid % nqt;
        h = bid / nqt;
    }
    const int kvh = h / (a.n_q / a.n_kv);
    const int HD = a.head_dim;
    const int qi = qt * 16 + c;
    const bool qok = qi < a.seq_q;
    const bool qfull = qt * 16 + 16 <= a.seq_q;  // every query of the tile exists
    float* Ks = smem + wave * C::TILE;
    float* Vs = Ks + KT * SK;

    float qreg[QS];
#pragma unroll
    for (int s = 0; s < QS; s += 4) {
        const int d = g * QS + s;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (qok && d < HD) v = *reinterpret_cast<const float4*>(a.Q + (size_t)qi * a.ldq + h * HD + d);
        qreg[s] = v.x;
        qreg[s + 1] = v.y;
        qreg[s + 2] = v.z;
        qreg[s + 3] = v.w;
    }

    const float scale = a.scale;
    const int mk = a.mask_kind;
    const int qg = (MKC == 3 && qok) ? a.q_group[qi] : 0;
    const int G = a.n_groups;
    // small group tables live in LDS, so the per-key test is an LDS read. The
    // main loop reads the table through `al` (derived from the shared array,
    // so its reads compile to ds_read_u8) or straight from global memory; one
    // pointer that could be either compiles to flat loads, whose waits
    // (vmcnt(0) as well) also drain the next key tile's prefetch.
    const bool allow_lds = MKC == 3 && G * G <= C::ALLOW;
    const uint8_t* al = reinterpret_cast<const uint8_t*>(smem) + C::MAIN;
    if (allow_lds) {
        uint8_t* alw = reinterpret_cast<uint8_t*>(smem) + C::MAIN;
        for (int i = tid; i < G * G; i += W * 64) alw[i] = a.allow[i];
        __syncthreads();
    }

    // keys past kv_end are blocked for every query of the block (causal bound)
    int kv_end = a.seq_k;
    if (mk == 2) {
        const int qlast = (qt * 16 + 16 < a.seq_q ? qt * 16 + 16 : a.seq_q) - 1;
        const int e = qlast + a.causal_offset + 1;
        kv_end = e < 0 ? 0 : (e < kv_end ? e : kv_end);
    }

    const bool vec_kg = MKC == 3 && (reinterpret_cast<uintptr_t>(a.k_group) & 3) == 0;
    const bool vec_mask = MKC == 1 && (reinterpret_cast<uintptr_t>(a.mask) & 15) == 0 && (a.ldm & 3) == 0;

    // this lane's share of a tile load: float4 number e = lane + 64 * i of the
    // KT x HDP/4 tile is row e / (HDP/4), dims 4 * (e % (HDP/4))
    float4 kr[F4], vr[F4];
    // with the tile: the mask data of the lane's keys kv0 + 16 kt + 4 g + r
    // (dense mask values or key groups), so the masking step waits on nothing.
    // A run of 4 key groups read as one word stays packed (gword) until the
    // tile is used: unpacking it here would make the wave wait for that load,
    // and with it for the whole K/V prefetch issued just before.
    float mnext[4 * NT];
    int gnext[4 * NT] = {};
    uint32_t gword[NT] = {};
    bool gpacked[NT] = {};
    auto gload = [&](int kv0, int end) {
        if (kv0 + KT <= end && HD == HDP) {  // wave-uniform: every row and column is in range
#pragma unroll
            for (int i = 0; i < F4; i++) {
                const int e = lane + 64 * i, row = e / (HDP / 4), d = 4 * (e % (HDP / 4));
                const int j = kv0 + row;
                kr[i] = *reinterpret_cast<const float4*>(a.K + (size_t)j * a.ldk + kvh * HD + d);
                vr[i] = *reinterpret_cast<const float4*>(a.V + (size_t)j * a.ldv + kvh * HD + d);
            }
        } else {
#pragma unroll
            for (int i = 0; i < F4; i++) {
                const int e = lane + 64 * i, row = e / (HDP / 4), d = 4 * (e % (HDP / 4));
                const int j = kv0 + row;
                kr[i] = vr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (j < end && d < HD) {
                    kr[i] = *reinterpret_cast<const float4*>(a.K + (size_t)j * a.ldk + kvh * HD + d);
                    vr[i] = *reinterpret_cast<const float4*>(a.V + (size_t)j * a.ldv + kvh * HD + d);
                }
            }
        }
        if (!KD) return;
        // a lane's keys come in runs of 4 consecutive (4 g .. 4 g + 3 of each
        // 16): whole in-range runs take one 4-byte group load or one float4
        // mask load when the table allows it
#pragma unroll
        for (int kt = 0; kt < NT; kt++) {
            const int j0 = kv0 + kt * 16 + 4 * g;
            if (MKC == 3) gpacked[kt] = j0 + 4 <= end && vec_kg;
            if (MKC == 3 && j0 + 4 <= end && vec_kg) {
                gword[kt] = *reinterpret_cast<const uint32_t*>(a.k_group + j0);
            } else if (MKC == 1 && j0 + 4 <= end && vec_mask) {
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (qok) v = *reinterpret_cast<const float4*>(a.mask + (size_t)qi * a.ldm + j0);
                mnext[kt * 4] = v.x;
                mnext[kt * 4 + 1] = v.y;
                mnext[kt * 4 + 2] = v.z;
                mnext[kt * 4 + 3] = v.w;
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int j = j0 + r;
                    mnext[kt * 4 + r] = 0.0f;
                    gnext[kt * 4 + r] = 0;
                    if (j < end) {
                        if (MKC == 1 && qok) mnext[kt * 4 + r] = a.mask[(size_t)qi * a.ldm + j];
                        else if (MKC == 3) gnext[kt * 4 + r] = a.k_group[j];
                    }
                }
            }
        }
    };
    auto lstore = [&]() {
#pragma unroll
        for (int i = 0; i < F4; i++) {
            const int e = lane + 64 * i, row = e / (HDP / 4), d = 4 * (e % (HDP / 4));
            *reinterpret_cast<float4*>(Ks + row * SK + d) = kr[i];
            *reinterpret_cast<float4*>(Vs + row * SK + d) = vr[i];
        }
    };

    float m = -INFINITY, lsum = 0.0f;
    v4f oacc[DT];
#pragma unroll
    for (int i = 0; i < DT; i++) oacc[i] = v4f{0.f, 0.f, 0.f, 0.f};

    const int nkt = (kv_end + KT - 1) / KT;
    if (wave < nkt) gload(wave * KT, a.seq_k);
    for (int t = wave; t < nkt; t += W) {
        const int kv0 = t * KT;
        lstore();
        float mcur[4 * NT];
        int gcur[4 * NT];
        if (KD) {
#pragma unroll
            for (int x = 0; x < 4 * NT; x++) {
                mcur[x] = mnext[x];
                gcur[x] = gpacked[x >> 2] ? (int)((gword[x >> 2] >> (8 * (x & 3))) & 0xffu) : gnext[x];
            }
        }
        wave_lds_sync();
        if (t + W < nkt) gload((t + W) * KT, a.seq_k);  // next tile, under this one's math

        // group masks: which of this lane's scores the table blocks, decided
        // before the products; a tile the table blocks for every query of the
        // wave adds p = 0 everywhere and leaves (m, l, O) as they are, so it
        // is skipped (Octo's later timesteps for earlier queries)
        bool mblk[4 * NT];
        if (MKC == 3) {
            bool live = false;
            if (allow_lds) {
#pragma unroll
                for (int x = 0; x < 4 * NT; x++) {
                    const int j = kv0 + (x >> 2) * 16 + 4 * g + (x & 3);
                    const bool b = !qok || j >= kv_end || !al[qg * G + gcur[x]];
                    mblk[x] = b;
                    live = live || !b;
                }
            } else {
#pragma unroll
                for (int x = 0; x < 4 * NT; x++) {
                    const int j = kv0 + (x >> 2) * 16 + 4 * g + (x & 3);
                    const bool b = !qok || j >= kv_end || !a.allow[qg * G + gcur[x]];
                    mblk[x] = b;
                    live = live || !b;
                }
            }
            if (!__any(live)) continue;
        }

        v4f sacc[NT];
#pragma unroll
        for (int kt = 0; kt < NT; kt++) {
            sacc[kt] = v4f{0.f, 0.f, 0.f, 0.f};
            const float* krow = Ks + (kt * 16 + c) * SK + g * QS;
#pragma unroll
            for (int s = 0; s < QS; s += 4) {
                const float4 kv = *reinterpret_cast<const float4*>(krow + s);
                sacc[kt] = mfma_f32(kv.x, qreg[s], sacc[kt]);
                sacc[kt] = mfma_f32(kv.y, qreg[s + 1], sacc[kt]);
                sacc[kt] = mfma_f32(kv.z, qreg[s + 2], sacc[kt]);
                sacc[kt] = mfma_f32(kv.w, qreg[s + 3], sacc[kt]);
            }
        }

        // scale, mask, tile max; a whole tile of keys for a whole query tile
        // with no mask (wave-uniform) only scales
        float mt = -INFINITY;
        if (MKC == 0 && mk == 0 && qfull && kv0 + KT <= kv_end) {
#pragma unroll
            for (int kt = 0; kt < NT; kt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float x = sacc[kt][r] * scale;
                    sacc[kt][r] = x;
                    mt = fmaxf(mt, x);
                }
        } else
#pragma unroll
        for (int kt = 0; kt < NT; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int j = kv0 + kt * 16 + 4 * g + r;
                float x = sacc[kt][r] * scale;
                bool blocked;
                if (MKC == 3) {
                    blocked = mblk[kt * 4 + r];
                } else if (MKC == 1) {
                    const float mv = mcur[kt * 4 + r];
                    blocked = !qok || j >= kv_end || mv == -FLT_MAX;
                    if (!blocked) x = x + mv;
                } else {
                    blocked = !qok || j >= kv_end || (mk == 2 && j > qi + a.causal_offset);
                }
                x = blocked ? -INFINITY : x;
                sacc[kt][r] = x;
                mt = fmaxf(mt, x);
            }
        mt = rows_max(mt);
        const float mnew = fmaxf(m, mt);

        float alpha = 1.0f;
        if (mnew == -INFINITY) {
#pragma unroll
            for (int kt = 0; kt < NT; kt++) sacc[kt] = v4f{0.f, 0.f, 0.f, 0.f};
        } else {
            // mnew == m gives alpha = exp2(0) = 1 exactly
            alpha = mnew == m ? 1.0f : fast_exp2((m - mnew) * kLog2e);
            float ps = 0.0f;
#pragma unroll
            for (int kt = 0; kt < NT; kt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float p = fast_exp2((sacc[kt][r] - mnew) * kLog2e);
                    sacc[kt][r] = p;
                    ps += p;
                }
            lsum = lsum * alpha + ps;
            m = mnew;
        }
        // the accumulators are rescaled only when some query's running max
        // moved (multiplying by alpha = 1 changes nothing)
        if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int dt = 0; dt < DT; dt++) oacc[dt] *= alpha;
        }
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
#pragma unroll
            for (int kt = 0; kt < NT; kt++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    oacc[dt] = mfma_f32(Vs[(kt * 16 + 4 * g + r) * SK + dt * 16 + c], sacc[kt][r], oacc[dt]);
        }
        wave_lds_sync();  // this tile's reads are done before the next lstore
    }

    lsum = rows_sum(lsum);

    // merge the waves' partial states: m*, then sum_w e^(m_w - m*) (l_w, O_w)
    __syncthreads();
    float* Mm = smem;               // [W][16]
    float* Ml = smem + 16 * W;      // [W][16]
    float* Mo = smem + 32 * W;      // [W][16][MO]
    if (g == 0) {
        Mm[wave * 16 + c] = m;
        Ml[wave * 16 + c] = lsum;
    }
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
        *reinterpret_cast<float4*>(Mo + (wave * 16 + c) * C::MO + dt * 16 + 4 * g) =
            make_float4(oacc[dt][0], oacc[dt][1], oacc[dt][2], oacc[dt][3]);
    __syncthreads();
    // every wave's (m, l) for this lane's query, in registers: the uniform pass
    // below reuses this LDS for V tiles
    float mw[W], lw[W], mstar = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; w++) {
        mw[w] = Mm[w * 16 + c];
        lw[w] = Ml[w * 16 + c];
        mstar = fmaxf(mstar, mw[w]);
    }
    const bool masked = qok && mstar == -INFINITY;
    // rows with every key blocked: uniform mean of V over all seq_k keys
    // (attn_uniform_row); the waves sum V over their tiles with p = 1
    if (__syncthreads_or(masked)) {
        // a row that is not masked keeps its softmax partial (it adds p = 0 below)
        if (masked)
#pragma unroll
            for (int i = 0; i < DT; i++) oacc[i] = v4f{0.f, 0.f, 0.f, 0.f};
        const int nall = (a.seq_k + KT - 1) / KT;
        for (int t = wave; t < nall; t += W) {
            const int kv0 = t * KT;
            gload(kv0, a.seq_k);
            lstore();
            wave_lds_sync();
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int kt = 0; kt < NT; kt++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int j = kv0 + kt * 16 + 4 * g + r;
                        const float p = (masked && j < a.seq_k) ? 1.0f : 0.0f;
                        oacc[dt] = mfma_f32(Vs[(kt * 16 + 4 * g + r) * SK + dt * 16 + c], p, oacc[dt]);
                    }
            wave_lds_sync();
        }
        __syncthreads();
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
            *reinterpret_cast<float4*>(Mo + (wave * 16 + c) * C::MO + dt * 16 + 4 * g) =
                make_float4(oacc[dt][0], oacc[dt][1], oacc[dt][2], oacc[dt][3]);
        __syncthreads();
    }
    // wave w writes the 16-dim output slices w, w + W, ... (every wave holds
    // all (m, l) already; the sums over waves run in the same order for each)
    if (wave >= DT || !qok) return;

    float f[W], l = 0.0f;
#pragma unroll
    for (int w = 0; w < W; w++) {
        f[w] = masked ? 1.0f : (mw[w] == -INFINITY ? 0.0f : fast_exp2((mw[w] - mstar) * kLog2e));
        l += f[w] * lw[w];
    }
    const float inv = masked ? 1.0f / (float)a.seq_k : 1.0f / l;
    for (int dt = wave; dt < DT; dt += W) {
        const int d = dt * 16 + 4 * g;
        if (d < HD) {
            float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int w = 0; w < W; w++) {
                const float4 v = *reinterpret_cast<const float4*>(Mo + (w * 16 + c) * C::MO + d);
                o.x += f[w] * v.x;
                o.y += f[w] * v.y;
                o.z += f[w] * v.z;
                o.w += f[w] * v.w;
            }
            o.x *= inv;
            o.y *= inv;
            o.z *= inv;
            o.w *= inv;
            *reinterpret_cast<float4*>(a.out + (size_t)qi * a.ldo + h * HD + d) = o;
        }
    }
}

template <int HDP, int KT, int W, int MKC>
void launch_kd(const AttnArgs& a, hipStream_t st) {
    using C = AttnCfg<HDP, KT, W>;
    static const bool attr = [] {
        if (C::LDS > 65536)
            VLA_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_fwd<HDP, KT, W, MKC>),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS));
        return true;
    }();
    (void)attr;
    attn_fwd<HDP, KT, W, MKC><<<dim3((a.seq_q + 15) / 16, a.n_q), W * 64, C::LDS, st>>>(a);
}

template <int HDP, int KT, int W>
void launch_w(const AttnArgs& a, hipStream_t st) {
    if (a.mask_kind == 1) launch_kd<HDP, KT, W, 1>(a, st);
    else if (a.mask_kind == 3) launch_kd<HDP, KT, W, 3>(a, st);
    else launch_kd<HDP, KT, W, 0>(a, st);
}

// VLA_HIP_ATTN_W=<1|2|4|8> forces the waves per block (A/B runs; the values
// only change by fp32 summation order across waves).
int forced_waves() {
    static const int w = [] {
        const char* e = std::getenv("VLA_HIP_ATTN_W");
        const int v = e ? std::atoi(e) : 0;
        return v == 1 || v == 2 || v == 4 || v == 8 ? v : 0;
    }();
    return w;
}

// W: enough waves that each walks a few key tiles, capped at WMAX (LDS).
template <int HDP, int KT, int WMAX>
void run_attn(const AttnArgs& a, hipStream_t st) {
    int kv = a.seq_k;
    if (a.mask_kind == 2) {  // keys no query of the problem can see are never walked
        const int e = a.seq_q + a.causal_offset;
        kv = e < 1 ? 1 : (e < kv ? e : kv);
    }
    int tiles = (kv + KT - 1) / KT;
    // grids of 1.5+ blocks per CU (Octo's 658-690 tokens x 12 heads): 4 waves,
    // so two blocks share a CU and hide each other's load latency (measured
    // 1.268 -> 1.235 ms and 1.457 -> 1.335 ms per Octo forward); smaller grids
    // (ACT, SmolVLA) keep 8 waves per block (their latency grew with 4)
    const long blocks = (long)((a.seq_q + 15) / 16) * a.n_q;
    if (blocks >= 384 && tiles > 4) tiles = 4;
    if (const int fw = forced_waves()) tiles = fw;
    if (tiles <= 1) launch_w<HDP, KT, 1>(a, st);
    else if (tiles <= 2 || WMAX == 2) launch_w<HDP, KT, 2>(a, st);
    else if (tiles <= 4 || WMAX == 4) launch_w<HDP, KT, (WMAX < 4 ? WMAX : 4)>(a, st);
    else launch_w<HDP, KT, WMAX>(a, st);
    VLA_LAUNCH_CHECK();
}

}  // namespace

void launch_attention(const AttnArgs& a, hipStream_t st) {
    VLA_REQUIRE(a.seq_q >= 0 && a.seq_k > 0 && a.n_q > 0 && a.n_kv > 0,
                "attention: need seq_q >= 0, seq_k > 0, n_q > 0, n_kv > 0");
    VLA_REQUIRE(a.n_q % a.n_kv == 0, "attention: n_q must be a multiple of n_kv");
    VLA_REQUIRE(a.head_dim > 0 && a.head_dim <= 256 && a.head_dim % 4 == 0,
                "attention: head_dim must be a multiple of 4 in [4, 256]");
    VLA_REQUIRE(a.ldq % 4 == 0 && a.ldk % 4 == 0 && a.ldv % 4 == 0 && a.ldo % 4 == 0,
                "attention: row strides must be multiples of 4 floats");
    VLA_REQUIRE(aligned(a.Q, 16) && aligned(a.K, 16) && aligned(a.V, 16) && aligned(a.out, 16),
                "attention: Q, K, V and out must be 16-byte aligned");
    VLA_REQUIRE(a.ldq >= a.n_q * a.head_dim && a.ldo >= a.n_q * a.head_dim &&
                    a.ldk >= a.n_kv * a.head_dim && a.ldv >= a.n_kv * a.head_dim,
                "attention: row stride shorter than heads * head_dim");
    VLA_REQUIRE(a.mask_kind >= 0 && a.mask_kind <= 3, "attention: unknown mask kind");
    VLA_REQUIRE(a.mask_kind != 1 || (a.mask && a.ldm >= a.seq_k), "attention: dense mask missing");
    VLA_REQUIRE(a.mask_kind != 3 || (a.q_group && a.k_group && a.allow && a.n_groups > 0 &&
                                     a.n_groups <= 256),
                "attention: group mask needs q_group, k_group, allow and 1..256 groups");
    if (a.seq_q == 0) return;
    if (a.head_dim <= 64)
        run_attn<64, 16, 8>(a, st);
    else if (a.head_dim <= 128)
        run_attn<128, 32, 4>(a, st);
    else
        run_attn<256, 16, 4>(a, st);
}

}  // namespace hip
}  // namespace vla
