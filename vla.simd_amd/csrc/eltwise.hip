// eltwise.hip - token-wise norms, RoPE and elementwise activations on gfx950.
//
// LayerNorm / RMSNorm follow src/hal/common/norms.cpp:19-35 and 69-97: per row
// the mean, variance and sum of squares accumulate in double (fp64 is a full
// rate path on CDNA4, and these kernels are HBM-bound), inv is computed in
// double and rounded once to float, and the output is formed in float from
// (float)(x - mean) exactly as the reference does. One wave64 owns a row and
// each lane reads and writes the same elements, so out may alias x (ACT calls
// layernorm(x, x), src/models/act/act_transformer.cpp:259).
//
// RoPE NeoX follows norms.cpp:37-67: theta_i = pos * base^(-2i/d) built by the
// same repeated double multiplication, double cos/sin, and the rotated pair
// formed in double then rounded to float.
//
// Activations are the device functions in act.h (also used by the GEMM
// epilogue). Every kernel here reads its input once and writes once.

#include "act.h"
#include "common.h"
#include "quant_row.h"
#include "rope.h"
#include "rowop.h"

namespace vla {
namespace hip {
namespace {


__global__ __launch_bounds__(256) void layernorm_kernel(float* out, const float* x, const float* w,
                                                        const float* b, int rows, int H, float eps) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* xr = x + (size_t)row * H;
    float* orow = out + (size_t)row * H;

    double s = 0.0;
    for (int k = lane; k < H; k += 64) s += (double)xr[k];
    const double mean = wave_sum_f64(s) / H;
    double v = 0.0;
    for (int k = lane; k < H; k += 64) {
        const double d = (double)xr[k] - mean;
        v += d * d;
    }
    const double var = wave_sum_f64(v);
    const float inv = (float)(1.0 / sqrt(var / H + (double)eps));
    for (int k = lane; k < H; k += 64) {
        const float c = (float)((double)xr[k] - mean);
        orow[k] = b ? fmaf(c * inv, w[k], b[k]) : c * inv * w[k];
    }
}

__global__ __launch_bounds__(256) void rmsnorm_kernel(float* out, const float* x, const float* w,
                                                      int rows, int H, float eps) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* xr = x + (size_t)row * H;
    float* orow = out + (size_t)row * H;
    double ss = 0.0;
    for (int k = lane; k < H; k += 64) {
        const double d = (double)xr[k];
        ss += d * d;
    }
    ss = wave_sum_f64(ss);
    const float inv = (float)(1.0 / sqrt(ss / H + (double)eps));
    for (int k = lane; k < H; k += 64) orow[k] = xr[k] * inv * w[k];
}

// layernorm_kernel / rmsnorm_kernel for rows of at most 64 J floats: the
// lane's elements (lane + 64 j, the same as the loops above visit) and its
// weights are loaded once, all in flight together, and the sums run in the
// same order, so the outputs are the loop kernels' bit for bit (the loops
// wait for each load before issuing the next). out may alias x.
template <int J>
__global__ __launch_bounds__(256) void layernorm_reg_kernel(float* out, const float* x, const float* w,
                                                            const float* b, int rows, int H, float eps) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* xr = x + (size_t)row * H;
    float* orow = out + (size_t)row * H;
    float xv[J], wv[J], bv[J];
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int k = lane + 64 * j;
        xv[j] = k < H ? xr[k] : 0.0f;
        wv[j] = k < H ? w[k] : 0.0f;
        bv[j] = b && k < H ? b[k] : 0.0f;
    }
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < J; j++)
        if (lane + 64 * j < H) s += (double)xv[j];
    const double mean = wave_sum_f64(s) / H;
    double v = 0.0;
#pragma unroll
    for (int j = 0; j < J; j++)
        if (lane + 64 * j < H) {
            const double d = (double)xv[j] - mean;
            v += d * d;
        }
    const double var = wave_sum_f64(v);
    const float inv = (float)(1.0 / sqrt(var / H + (double)eps));
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int k = lane + 64 * j;
        if (k < H) {
            const float c = (float)((double)xv[j] - mean);
            orow[k] = b ? fmaf(c * inv, wv[j], bv[j]) : c * inv * wv[j];
        }
    }
}

template <int J>
__global__ __launch_bounds__(256) void rmsnorm_reg_kernel(float* out, const float* x, const float* w, int rows,
                                                          int H, float eps) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* xr = x + (size_t)row * H;
    float* orow = out + (size_t)row * H;
    float xv[J], wv[J];
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int k = lane + 64 * j;
        xv[j] = k < H ? xr[k] : 0.0f;
        wv[j] = k < H ? w[k] : 0.0f;
    }
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < J; j++)
        if (lane + 64 * j < H) {
            const double d = (double)xv[j];
            ss += d * d;
        }
    ss = wave_sum_f64(ss);
    const float inv = (float)(1.0 / sqrt(ss / H + (double)eps));
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int k = lane + 64 * j;
        if (k < H) orow[k] = xv[j] * inv * wv[j];
    }
}

template <int ACT>
__global__ __launch_bounds__(256) void act_kernel(float* x, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        x[i] = apply_act<ACT>(x[i]);
}

__global__ __launch_bounds__(256) void silu_gate_kernel(float* out, const float* g, const float* u,
                                                        int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = act_silu_gate(g[i], u[i]);
}

// silu_gate over a [rows, cols] block whose g and u rows are strided (the
// gate|up halves of one concatenated GEMM output)
__global__ __launch_bounds__(256) void silu_gate_rows_kernel(float* out, int ldo, const float* g,
                                                             int ldg, const float* u, int ldu,
                                                             int cols) {
    const int r = blockIdx.y;
    for (int c = blockIdx.x * 256 + threadIdx.x; c < cols; c += gridDim.x * 256)
        out[(size_t)r * ldo + c] = act_silu_gate(g[(size_t)r * ldg + c], u[(size_t)r * ldu + c]);
}

__global__ __launch_bounds__(256) void add_kernel(float* out, const float* a, const float* b,
                                                  int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = a[i] + b[i];
}

// one thread per (token, head, pair index i); cos/sin of (token, i) from a
// table built on the host exactly as rope_neox builds its per-token table
__global__ __launch_bounds__(256) void rope_table_kernel(float* x, int ld, const double* cs, int seq,
                                                         int n_heads, int half) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= seq * n_heads * half) return;
    const int i = idx % half, hh = (idx / half) % n_heads, t = idx / (half * n_heads);
    const double c = cs[((size_t)t * half + i) * 2], s = cs[((size_t)t * half + i) * 2 + 1];
    float* v = x + (size_t)t * ld + hh * 2 * half;
    const float x0 = v[i], x1 = v[i + half];
    v[i] = rope_lo(x0, x1, c, s);
    v[i + half] = rope_hi(x0, x1, c, s);
}

// one thread per (token, pair index i); loops over heads
__global__ __launch_bounds__(256) void rope_kernel(float* x, int ld, const int32_t* pos, int seq,
                                                   int n_heads, int head_dim, double theta_scale) {
    const int half = head_dim / 2;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= seq * half) return;
    const int t = idx / half, i = idx % half;
    double theta = (double)pos[t];
    for (int j = 0; j < i; j++) theta *= theta_scale;
    const double c = cos(theta), s = sin(theta);
    float* row = x + (size_t)t * ld;
    for (int hh = 0; hh < n_heads; hh++) {
        float* v = row + hh * head_dim;
        const float x0 = v[i], x1 = v[i + half];
        v[i] = rope_lo(x0, x1, c, s);
        v[i + half] = rope_hi(x0, x1, c, s);
    }
}

// one block per row segment of 1024 floats
__global__ __launch_bounds__(256) void copy_rows_kernel(float* dst, int ldd, const float* src,
                                                        int lds, int cols) {
    const int r = blockIdx.y;
    const int c = blockIdx.x * 1024 + threadIdx.x;
#pragma unroll
    for (int j = 0; j < 4; j++)
        if (c + 256 * j < cols) dst[(size_t)r * ldd + c + 256 * j] = src[(size_t)r * lds + c + 256 * j];
}

// One wave per row; the row lives in registers (NV float4 per lane, element
// 4 * lane + 256 * i), so the norm statistics, the fp32 result and the
// absmax of the quantizer all come from one read of the row. The norms
// accumulate in double as layernorm_kernel / rmsnorm_kernel do.
template <int OP, int NV>
__global__ __launch_bounds__(256) void rowq_kernel(RowQArgs a) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.rows) return;  // wave-uniform
    const int H = a.H;
    // the second output's addend, in flight with the row (zero past H)
    float4 addv[NV];
    if (a.add) {
        const float* ar = a.add + (size_t)row * a.ld_add;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int k = 4 * lane + 256 * i;
            addv[i] = k < H ? *reinterpret_cast<const float4*>(ar + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    float4 y[NV];
    rowop_apply<OP, NV>(y, a.x + (size_t)row * a.ldx, OP == 3 ? a.u + (size_t)row * a.ldu : nullptr, a.w, a.b,
                        a.eps, H, lane);

    // y -> out (fp32) and q (int8); then y + add -> out2 and q2
#pragma unroll
    for (int pass = 0; pass < 2; pass++) {
        float* out = pass ? a.out2 : a.out;
        int8_t* q = pass ? a.q2 : a.q;
        if (pass == 1) {
            if (!a.add) break;
#pragma unroll
            for (int i = 0; i < NV; i++) {
                const int k = 4 * lane + 256 * i;
                if (k < H) {
                    const float4 p = addv[i];
                    y[i] = make_float4(y[i].x + p.x, y[i].y + p.y, y[i].z + p.z, y[i].w + p.w);
                }
            }
        }
        if (out) {
            float* orow = out + (size_t)row * (pass ? a.ldo2 : a.ldo);
#pragma unroll
            for (int i = 0; i < NV; i++) {
                const int k = 4 * lane + 256 * i;
                if (k < H) *reinterpret_cast<float4*>(orow + k) = y[i];
            }
        }
        if (q) {
            const float s = rowop_scale<NV>(y, H, lane);
            const float inv = 1.0f / s;
            if (lane == 0) (pass ? a.qs2 : a.qs)[row] = s;
            if (a.q_panel) {
                // panel layout (common.h): word k of the row at (k / 64) * mp * 64 + row * 64 + k % 64
                const size_t pstride = (size_t)panel_rows(a.rows) * 64;
                int8_t* qr = q + (size_t)row * 64;
#pragma unroll
                for (int i = 0; i < NV; i++) {
                    const int k = 4 * lane + 256 * i;
                    if (k < H) *reinterpret_cast<uint32_t*>(qr + (k >> 6) * pstride + (k & 63)) = q8x4(y[i], inv);
                }
                for (int k = H + 4 * lane; k < ((H + 63) & ~63); k += 256)
                    *reinterpret_cast<uint32_t*>(qr + (k >> 6) * pstride + (k & 63)) = 0u;
            } else {
                const int ldq = pass ? a.ldq2 : a.ldq;
                int8_t* qr = q + (size_t)row * ldq;
#pragma unroll
                for (int i = 0; i < NV; i++) {
                    const int k = 4 * lane + 256 * i;
                    if (k < H) *reinterpret_cast<uint32_t*>(qr + k) = q8x4(y[i], inv);
                }
                for (int k = H + 4 * lane; k < ldq; k += 256) *reinterpret_cast<uint32_t*>(qr + k) = 0u;
            }
        }
    }
}

// rowq_kernel for the element-wise row ops (0 identity, 3 silu_gate) without
// an add: a whole 256-thread block per row, so a 2048-wide SiLU-gate row is
// 8 elements per lane instead of 32 and the rows' expf / divisions spread
// over rows x 4 waves. Thread t holds elements 4 t + 1024 i. The values are
// the single-wave kernel's: the element ops are the same functions and the
// row max does not depend on the reduction order.
template <int OP, int NV>
__global__ __launch_bounds__(256) void rowq_wide_kernel(RowQArgs a) {
    static_assert(OP == 0 || OP == 3, "element-wise row ops only");
    __shared__ float red[4];
    const int row = blockIdx.x, t = threadIdx.x, H = a.H;
    const float* xr = a.x + (size_t)row * a.ldx;
    const float* ur = OP == 3 ? a.u + (size_t)row * a.ldu : nullptr;
    float4 y[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int k = 4 * t + 1024 * i;
        y[i] = k < H ? *reinterpret_cast<const float4*>(xr + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (OP == 3) {
        // the up row loads all in flight before the first use
        float4 u[NV];
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int k = 4 * t + 1024 * i;
            u[i] = k < H ? *reinterpret_cast<const float4*>(ur + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int k = 4 * t + 1024 * i;
            if (k < H)
                y[i] = make_float4(act_silu_gate(y[i].x, u[i].x), act_silu_gate(y[i].y, u[i].y),
                                   act_silu_gate(y[i].z, u[i].z), act_silu_gate(y[i].w, u[i].w));
        }
    }
    if (a.out) {
        float* orow = a.out + (size_t)row * a.ldo;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int k = 4 * t + 1024 * i;
            if (k < H) *reinterpret_cast<float4*>(orow + k) = y[i];
        }
    }
    if (!a.q) return;  // block-uniform
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++)
        if (4 * t + 1024 * i < H)
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(y[i].x), fabsf(y[i].y)), fmaxf(fabsf(y[i].z), fabsf(y[i].w))));
    amax = wave_max_f32(amax);
    if ((t & 63) == 0) red[t >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s = row_scale(amax), inv = 1.0f / s;
    if (t == 0) a.qs[row] = s;
    if (a.q_panel) {
        const size_t pstride = (size_t)panel_rows(a.rows) * 64;
        int8_t* qr = a.q + (size_t)row * 64;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int k = 4 * t + 1024 * i;
            if (k < H) *reinterpret_cast<uint32_t*>(qr + (k >> 6) * pstride + (k & 63)) = q8x4(y[i], inv);
        }
        for (int k = H + 4 * t; k < ((H + 63) & ~63); k += 1024)
            *reinterpret_cast<uint32_t*>(qr + (k >> 6) * pstride + (k & 63)) = 0u;
    } else {
        int8_t* qr = a.q + (size_t)row * a.ldq;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int k = 4 * t + 1024 * i;
            if (k < H) *reinterpret_cast<uint32_t*>(qr + k) = q8x4(y[i], inv);
        }
        for (int k = H + 4 * t; k < a.ldq; k += 1024) *reinterpret_cast<uint32_t*>(qr + k) = 0u;
    }
}

template <int OP>
void launch_rowq_op(const RowQArgs& a, hipStream_t st) {
    if constexpr (OP == 0 || OP == 3) {
        // wide rows of an element-wise op (and no second output): a block per row
        if (!a.add && a.H >= 1024) {
            const int nw = (a.H + 1023) / 1024;
            if (nw <= 1) rowq_wide_kernel<OP, 1><<<a.rows, 256, 0, st>>>(a);
            else if (nw <= 2) rowq_wide_kernel<OP, 2><<<a.rows, 256, 0, st>>>(a);
            else rowq_wide_kernel<OP, 4><<<a.rows, 256, 0, st>>>(a);
            return;
        }
    }
    const int nv = (a.H + 255) / 256;
    const dim3 grid((a.rows + 3) / 4), block(256);
    if (nv <= 1) rowq_kernel<OP, 1><<<grid, block, 0, st>>>(a);
    else if (nv <= 2) rowq_kernel<OP, 2><<<grid, block, 0, st>>>(a);
    else if (nv <= 4) rowq_kernel<OP, 4><<<grid, block, 0, st>>>(a);
    else if (nv <= 8) rowq_kernel<OP, 8><<<grid, block, 0, st>>>(a);
    else rowq_kernel<OP, 16><<<grid, block, 0, st>>>(a);
}

int grid_for(int64_t n) {
    const int64_t b = (n + 255) / 256;
    return (int)(b < 4096 ? (b > 0 ? b : 1) : 4096);
}

}  // namespace

void launch_layernorm(float* out, const float* x, const float* w, const float* b, int rows,
                      int hidden, float eps, hipStream_t st) {
    VLA_REQUIRE(rows >= 0 && hidden > 0, "layernorm: need rows >= 0 and hidden > 0");
    if (rows == 0) return;
    const int g = (rows + 3) / 4;
    if (hidden <= 256) layernorm_reg_kernel<4><<<g, 256, 0, st>>>(out, x, w, b, rows, hidden, eps);
    else if (hidden <= 512) layernorm_reg_kernel<8><<<g, 256, 0, st>>>(out, x, w, b, rows, hidden, eps);
    else if (hidden <= 1024) layernorm_reg_kernel<16><<<g, 256, 0, st>>>(out, x, w, b, rows, hidden, eps);
    else if (hidden <= 2048) layernorm_reg_kernel<32><<<g, 256, 0, st>>>(out, x, w, b, rows, hidden, eps);
    else layernorm_kernel<<<g, 256, 0, st>>>(out, x, w, b, rows, hidden, eps);
    VLA_LAUNCH_CHECK();
}

void launch_rmsnorm(float* out, const float* x, const float* w, int rows, int hidden, float eps,
                    hipStream_t st) {
    VLA_REQUIRE(rows >= 0 && hidden > 0, "rmsnorm: need rows >= 0 and hidden > 0");
    if (rows == 0) return;
    const int g = (rows + 3) / 4;
    if (hidden <= 256) rmsnorm_reg_kernel<4><<<g, 256, 0, st>>>(out, x, w, rows, hidden, eps);
    else if (hidden <= 512) rmsnorm_reg_kernel<8><<<g, 256, 0, st>>>(out, x, w, rows, hidden, eps);
    else if (hidden <= 1024) rmsnorm_reg_kernel<16><<<g, 256, 0, st>>>(out, x, w, rows, hidden, eps);
    else if (hidden <= 2048) rmsnorm_reg_kernel<32><<<g, 256, 0, st>>>(out, x, w, rows, hidden, eps);
    else rmsnorm_kernel<<<g, 256, 0, st>>>(out, x, w, rows, hidden, eps);
    VLA_LAUNCH_CHECK();
}

void launch_act(float* x, int64_t n, int act, hipStream_t st) {
    VLA_REQUIRE(n >= 0, "activation: n < 0");
    if (n == 0 || act == 0) return;
    switch (act) {
    case 1: act_kernel<1><<<grid_for(n), 256, 0, st>>>(x, n); break;
    case 2: act_kernel<2><<<grid_for(n), 256, 0, st>>>(x, n); break;
    case 3: act_kernel<3><<<grid_for(n), 256, 0, st>>>(x, n); break;
    case 4: act_kernel<4><<<grid_for(n), 256, 0, st>>>(x, n); break;
    default: throw ArgError("activation: unknown kind");
    }
    VLA_LAUNCH_CHECK();
}

void launch_silu_gate(float* out, const float* g, const float* u, int64_t n, hipStream_t st) {
    VLA_REQUIRE(n >= 0, "silu_gate: n < 0");
    if (n == 0) return;
    silu_gate_kernel<<<grid_for(n), 256, 0, st>>>(out, g, u, n);
    VLA_LAUNCH_CHECK();
}

void launch_silu_gate_rows(float* out, int ldo, const float* g, int ldg, const float* u, int ldu,
                           int rows, int cols, hipStream_t st) {
    VLA_REQUIRE(rows >= 0 && rows < 65536 && cols >= 0 && ldo >= cols && ldg >= cols && ldu >= cols,
                "silu_gate_rows: bad shape");
    if (rows == 0 || cols == 0) return;
    const int gx = (cols + 255) / 256 < 8 ? (cols + 255) / 256 : 8;
    silu_gate_rows_kernel<<<dim3(gx, rows), 256, 0, st>>>(out, ldo, g, ldg, u, ldu, cols);
    VLA_LAUNCH_CHECK();
}

void launch_add(float* out, const float* a, const float* b, int64_t n, hipStream_t st) {
    VLA_REQUIRE(n >= 0, "add: n < 0");
    if (n == 0) return;
    add_kernel<<<grid_for(n), 256, 0, st>>>(out, a, b, n);
    VLA_LAUNCH_CHECK();
}

void launch_copy_rows(float* dst, int ldd, const float* src, int lds, int rows, int cols,
                      hipStream_t st) {
    VLA_REQUIRE(rows >= 0 && cols >= 0 && ldd >= cols && lds >= cols, "copy_rows: bad shape");
    VLA_REQUIRE(rows < 65536, "copy_rows: too many rows");
    if (rows == 0 || cols == 0) return;
    copy_rows_kernel<<<dim3((cols + 1023) / 1024, rows), 256, 0, st>>>(dst, ldd, src, lds, cols);
    VLA_LAUNCH_CHECK();
}

void launch_rowq(const RowQArgs& a, hipStream_t st) {
    VLA_REQUIRE(a.op >= 0 && a.op <= 3, "rowq: unknown row op");
    VLA_REQUIRE(a.rows >= 0 && a.H > 0 && a.H % 4 == 0 && a.H <= 16 * 256,
                "rowq: rows must be >= 0 and H a multiple of 4 in [4, 4096]");
    VLA_REQUIRE(a.x && a.ldx >= a.H && a.ldx % 4 == 0 && aligned(a.x, 16), "rowq: x rows must be 16-byte aligned");
    VLA_REQUIRE(a.op == 0 || a.op == 3 || (a.w && aligned(a.w, 16) && (!a.b || aligned(a.b, 16))),
                "rowq: norm weights must be 16-byte aligned");
    VLA_REQUIRE(a.op != 3 || (a.u && a.ldu >= a.H && a.ldu % 4 == 0 && aligned(a.u, 16)),
                "rowq: silu_gate needs 16-byte aligned u rows");
    VLA_REQUIRE(!a.out || (a.ldo >= a.H && a.ldo % 4 == 0 && aligned(a.out, 16)), "rowq: bad out");
    VLA_REQUIRE(!a.q_panel || a.rows <= kPanelMaxRows, "rowq: the panel layout holds at most 128 rows");
    VLA_REQUIRE(!a.q || (a.qs && (a.q_panel || (a.ldq >= a.H && a.ldq % 4 == 0)) && aligned(a.q, 4)),
                "rowq: bad q");
    VLA_REQUIRE(!a.add || (a.ld_add >= a.H && a.ld_add % 4 == 0 && aligned(a.add, 16)), "rowq: bad add");
    VLA_REQUIRE(!a.out2 || (a.add && a.ldo2 >= a.H && a.ldo2 % 4 == 0 && aligned(a.out2, 16)),
                "rowq: bad out2");
    VLA_REQUIRE(!a.q2 || (a.add && a.qs2 && (a.q_panel || (a.ldq2 >= a.H && a.ldq2 % 4 == 0)) &&
                          aligned(a.q2, 4)),
                "rowq: bad q2");
    if (a.rows == 0) return;
    if (a.op == 0) launch_rowq_op<0>(a, st);
    else if (a.op == 1) launch_rowq_op<1>(a, st);
    else if (a.op == 2) launch_rowq_op<2>(a, st);
    else launch_rowq_op<3>(a, st);
    VLA_LAUNCH_CHECK();
}

void launch_rope_table(float* x, int ld, const double* cs, int seq, int n_heads, int head_dim,
                       hipStream_t st) {
    VLA_REQUIRE(seq >= 0 && n_heads > 0 && head_dim > 0 && head_dim % 2 == 0 && cs,
                "rope: need seq >= 0, n_heads > 0, an even head_dim and a table");
    VLA_REQUIRE(ld >= n_heads * head_dim, "rope: row stride shorter than heads * head_dim");
    if (seq == 0) return;
    const int n = seq * n_heads * (head_dim / 2);
    rope_table_kernel<<<(n + 255) / 256, 256, 0, st>>>(x, ld, cs, seq, n_heads, head_dim / 2);
    VLA_LAUNCH_CHECK();
}

void launch_rope_neox(float* x, int ld, const int32_t* pos, int seq, int n_heads, int head_dim,
                      float base, hipStream_t st) {
    VLA_REQUIRE(seq >= 0 && n_heads > 0 && head_dim > 0 && head_dim % 2 == 0,
                "rope_neox: need seq >= 0, n_heads > 0 and an even head_dim");
    VLA_REQUIRE(ld >= n_heads * head_dim, "rope_neox: row stride shorter than heads * head_dim");
    if (seq == 0) return;
    const double theta_scale = pow((double)base, -2.0 / head_dim);
    const int n = seq * (head_dim / 2);
    rope_kernel<<<(n + 255) / 256, 256, 0, st>>>(x, ld, pos, seq, n_heads, head_dim, theta_scale);
    VLA_LAUNCH_CHECK();
}

}  // namespace hip
}  // namespace vla
